#!/usr/bin/env python3
"""Reshard-repack benchmark on one MI355X.

Default workload: Llama-2-7B shape (6.74e9 params), bf16 params + fp32 main /
exp_avg / exp_avg_sq, world 8 simulated on one GPU, distributed optimizer with
40M-element buckets, TP1 PP1 DP8 -> TP4 PP1 DP2, emitting every target shard.

A step is one execution of the switch's copy plan (the copy kernel, after a
short pre-read of the plan's lookup tables) with
every source shard already resident in HBM.  Inputs are synthetic: seeded
values ~N(0, 0.02) for bf16 params, main = their exact upcast, exp_avg
~N(0, 1e-3), exp_avg_sq = |N(0, 1e-6)|.  The destination is checked
bit-exact against the generator after the timed steps.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints one JSON line.  ``value`` is payload throughput: bytes of model state
(bf16 params + fp32 optimizer state) delivered to the target layout per
second.  ``roofline.achieved`` is algorithmic HBM traffic per second: every
byte the plan reads plus every byte it writes (by default the bf16 params are
the rounding of the new fp32 main weights, written in the same pass, so a
parameter costs 12 bytes read and 14 written).
"""

import argparse
import json
import logging
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "reshard repack GB/s & ms (params+Adam state), Llama-2-7B TP1DP8→TP4DP2, 1 GPU"
HEADLINE = "llama2-7b-tp1dp8-tp4dp2"
HBM_PEAK_GBPS = 8000.0
SEED = 1234


def workloads():
    from elasticmegatron_amd import ParallelStrategy as PS
    from elasticmegatron_amd.resharding import model_spec as ms

    return {
        "llama2-7b-tp1dp8-tp4dp2": ("Llama-2-7B TP1PP1DP8 -> TP4PP1DP2, world 8, 40M buckets",
                                    ms.llama2_7b, PS(8, 1, 1), PS(8, 4, 1)),
        "tiny-llama2-tp2dp4-tp1dp8": ("tiny LLaMA-2 (2L h512) TP2DP4 -> TP1DP8, world 8",
                                      ms.tiny_llama2, PS(8, 2, 1), PS(8, 1, 1)),
        "tiny-llama2-tp1dp8-tp4dp2": ("tiny LLaMA-2 (2L h512) TP1DP8 -> TP4DP2, world 8",
                                      ms.tiny_llama2, PS(8, 1, 1), PS(8, 4, 1)),
        "llama3-8b-tp2pp2dp2-tp4pp1dp2": ("Llama-3-8B GQA TP2PP2DP2 -> TP4PP1DP2, world 8",
                                          ms.llama3_8b, PS(8, 2, 2), PS(8, 4, 1)),
        "llama3-8b-tp2pp2dp2-tp4pp1dp2-repad": ("Llama-3-8B GQA TP2PP2DP2 -> TP4PP1DP2, world 8, vocabulary "
                                                "re-padded 128256 -> 128512", ms.llama3_8b, PS(8, 2, 2),
                                                PS(8, 4, 1), True),
        "mixtral-4l-ep4-ep8": ("Mixtral-8x7B 4-layer slice EP4 (EDP2) -> EP8 (EDP1), world 8",
                               ms.mixtral_8x7b_slice, PS(8, 1, 1, expert_model_parallel_size=4),
                               PS(8, 1, 1, expert_model_parallel_size=8)),
        "llama2-7b-dp8-dp6": ("Llama-2-7B world 8 DP8 -> world 6 DP6", ms.llama2_7b, PS(8, 1, 1), PS(6, 1, 1)),
        "llama2-7b-cp2tp2dp2-tp4dp2": ("Llama-2-7B CP2TP2DP2 -> TP4DP2, world 8, 40M buckets", ms.llama2_7b,
                                       PS(8, 2, 1, context_parallel_size=2), PS(8, 4, 1)),
        "llama2-7b-groupzero-1-2": ("Llama-2-7B Group ZeRO instances 1 -> 2 (world 6 -> 12), fp32 only",
                                    ms.llama2_7b, PS(6, 1, 1),
                                    PS(12, 1, 1, num_distributed_optimizer_instances=2)),
        "llama2-7b-groupzero-2-1": ("Llama-2-7B Group ZeRO instances 2 -> 1 (world 12 -> 6), fp32 only",
                                    ms.llama2_7b, PS(12, 1, 1, num_distributed_optimizer_instances=2),
                                    PS(6, 1, 1)),
        "tiny-llama2-groupzero-1-2": ("tiny LLaMA-2 (2L h512) Group ZeRO instances 1 -> 2 (world 4 -> 8), fp32 only",
                                      ms.tiny_llama2, PS(4, 1, 1), PS(8, 1, 1, num_distributed_optimizer_instances=2)),
        "tiny-llama2-groupzero-2-1": ("tiny LLaMA-2 (2L h512) Group ZeRO instances 2 -> 1 (world 8 -> 4), fp32 only",
                                      ms.tiny_llama2, PS(8, 1, 1, num_distributed_optimizer_instances=2), PS(4, 1, 1)),
        # 182 GB per state: only a staged switch (--low-memory) fits it on one GPU.
        "llama2-13b-tp1dp8-tp4dp2": ("Llama-2-13B TP1PP1DP8 -> TP4PP1DP2, world 8, 40M buckets",
                                     ms.llama2_13b, PS(8, 1, 1), PS(8, 4, 1)),
        # 966 GB per state: one destination rank's share (--share-rank) is what one GPU runs.
        "llama2-70b-tp8pp4dp2-tp4pp4dp4": ("Llama-2-70B TP8PP4DP2 -> TP4PP4DP4, world 64, 40M buckets",
                                           ms.llama2_70b, PS(64, 8, 4), PS(64, 4, 4)),
    }


def metric_for(workload: str, desc: str) -> str:
    """The headline metric for the headline workload; any other line names its own switch."""
    if workload == HEADLINE:
        return METRIC
    return f"reshard repack GB/s & ms (params+Adam state), {desc}, 1 GPU"


SHAPE_KEYS = ("lanes", "units", "chunk_index", "warm_tables", "xcd_remap", "buffer_ops", "nontemporal",
              "persistent", "blocks_per_cu", "run")


def parse_shapes(text):
    """``--shape-sweep`` value: launch shapes separated by ``;``, each ``default`` or comma-separated
    ``key=int`` settings of emrs_tuning (unset keys keep their defaults)."""
    shapes = []
    for part in text.split(";"):
        part = part.strip()
        shape = {}
        if part and part != "default":
            for kv in part.split(","):
                key, sep, val = kv.partition("=")
                key = key.strip().replace("-", "_")
                if not sep or key not in SHAPE_KEYS:
                    raise argparse.ArgumentTypeError(f"bad launch-shape setting {kv!r}; keys: {', '.join(SHAPE_KEYS)}")
                try:
                    shape[key] = int(val)
                except ValueError:
                    raise argparse.ArgumentTypeError(f"launch-shape setting {kv!r} is not an integer") from None
        lanes, units = shape.get("lanes", 0) or 64, shape.get("units", 1)
        if lanes not in (64, 128, 256) or units not in (0, 1, 2, 4) or (units and 256 % (lanes * units)):
            raise argparse.ArgumentTypeError(f"launch shape {part!r}: lanes 64/128/256, units 0/1/2/4, "
                                             "lanes * units dividing 256")
        shapes.append(shape)
    return shapes


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default=HEADLINE)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-verify", action="store_true")
    ap.add_argument("--no-e2e", action="store_true", help="skip timing ElasticMegatronManager.reshard end to end")
    ap.add_argument("--no-copy-ceiling", action="store_true", help="skip the plain-copy reference launch")
    ap.add_argument("--tensors", action="store_true",
                    help="run the per-tensor plan (one buffer per stored tensor, as views into the arenas)")
    ap.add_argument("--placement-trials", type=int, default=0,
                    help="re-allocate the destination state this many times and time 5 launches each")
    ap.add_argument("--shape-sweep", type=parse_shapes, default=None,
                    help="time several launch shapes on the same allocations, in --rounds rounds, e.g. "
                         "'default;units=4,chunk_index=0;units=2'; prints one JSON line per workload")
    ap.add_argument("--rounds", type=int, default=3, help="rounds of --shape-sweep")
    ap.add_argument("--rank-shares", action="store_true",
                    help="time each destination rank's share of the plan on its own (the part one GPU "
                         "would run with one rank per GPU) beside the whole plan, on the same allocations")
    ap.add_argument("--share-rank", type=int, default=None,
                    help="run only this destination rank's share of the switch, on the tensors it touches "
                         "alone (allocated one per stored tensor): the part one GPU runs with one rank per GPU; "
                         "-1: every rank's share in turn")
    ap.add_argument("--bf16-source", choices=("cast", "copy"), default="cast",
                    help="cast: bf16 params = bf16(new main), fused into the main copy; copy: from source bf16")
    ap.add_argument("--lanes", type=int, default=0, choices=(0, 64, 128, 256),
                    help="one workgroup per piece of a chunk of 256 units: lanes per workgroup (0: the default, 64)")
    ap.add_argument("--units", type=int, default=1, choices=(0, 1, 2, 4),
                    help="16-byte units per lane (default 1; 0: a whole chunk per workgroup, 256 / lanes)")
    ap.add_argument("--chunk-index", type=int, default=1, choices=(0, 1),
                    help="1: each workgroup reads its segment from the plan's chunk table; 0: binary search")
    ap.add_argument("--warm-tables", type=int, default=1, choices=(0, 1),
                    help="1: read the chunk and segment tables just before each copy (with --chunk-index 1)")
    ap.add_argument("--persistent", type=int, default=0,
                    help="0: one workgroup per piece of a chunk; 1: persistent grid (--blocks-per-cu, --run)")
    ap.add_argument("--blocks-per-cu", type=int, default=0, help="persistent grid; 0: as many as can be resident")
    ap.add_argument("--nontemporal", type=int, default=1)
    ap.add_argument("--xcd-remap", type=int, default=1, choices=(0, 1, 2),
                    help="each XCD takes one contiguous eighth of the chunks: 1 in the persistent grid and for "
                         "plans of at least 2^19 chunks, 2 always, 0 never")
    ap.add_argument("--run", type=int, default=4,
                    help="persistent grid; 0: contiguous chunk run per workgroup; N: round-robin runs of 8N chunks")
    ap.add_argument("--megatron-buffers", action="store_true",
                    help="run the per-tensor plan on views of Megatron-shaped flat buffers (a DDP param buffer per "
                         "model shard, flat DP shards per rank, padding in place), allocated separately")
    ap.add_argument("--ipc", action="store_true",
                    help="the switch from another process's state: a child exports the source in granules "
                         "(--ipc-granule-bytes), this process maps them and reshards into its own arenas")
    ap.add_argument("--ipc-granule-bytes", type=int, default=1 << 30)
    ap.add_argument("--lost-ranks", type=lambda t: tuple(int(x) for x in t.split(",") if x), default=(),
                    help="Group-ZeRO workloads: time the switch with these source ranks' fp32 state poisoned and "
                         "read from another optimizer instance, beside the plain switch")
    ap.add_argument("--adopt", action="store_true",
                    help="Group-ZeRO workloads: time the switch between shared states (granules of "
                         "--ipc-granule-bytes) with instance 0 copied and with the new state taking it over, launch "
                         "and ElasticMegatronManager.reshard end to end")
    ap.add_argument("--shared-states", action="store_true",
                    help="with --low-memory: every state held in granules of --ipc-granule-bytes, as a state another "
                         "process can map")
    ap.add_argument("--low-memory", action="store_true",
                    help="time staged switches through ElasticMegatronManager(low_memory=True), alternating "
                         "directions: one optimizer kind per launch, arenas allocated and released as it goes")
    ap.add_argument("--copy-calibration-gib", type=float, default=0.0,
                    help="time a single contiguous copy of this many GiB instead (traffic calibration)")
    return ap.parse_args()


def cpu_baseline(spec, ls, src, dst, backup, a):
    """Oracle-1 (the reference's three-pass executor restated on CPU torch tensors) on every
    parameter of the switch, one parameter at a time, on all of the host's cores.

    Each parameter's source pieces are copied from the device state ``a`` (the seeded values;
    outside the timed region, as the reference's Timer scopes only the executor), then the
    oracle's passes for that parameter are timed.  The parameters' times add up to the whole
    switch, as the reference's loop over parameters does (transfer.py:291-341)."""
    import torch

    from oracle import model
    from oracle import transfer as oracle1
    from oracle.plan import Strat, dp_distributions, local_shape, tp_size

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    inv = model.inventory(spec)
    S, D = Strat.of(src), Strat.of(dst)
    sd, dd = dp_distributions(inv, S, spec), dp_distributions(inv, D, spec)
    space = ls.space
    total_t = total_b = copy_t = 0.0
    l0_t = l0_b = 0.0
    n_params = n_elems = 0
    for p in inv:
        pid = p["id"]
        if pid not in sd:
            continue
        vp = space.all_virtual_params[pid]
        shape = local_shape(p, tp_size(S, p))
        t0 = time.perf_counter()
        world = {pid: {h.rank: oracle1.OptInfo([t[h.offset:h.offset + h.hi - h.lo].cpu()
                                                for t in (a.main, a.exp_avg, a.exp_avg_sq)], (h.lo, h.hi), shape)
                       for h in ls.fp32_holders(vp)}}
        t1 = time.perf_counter()
        if backup is None:
            dw, dbf, _ = oracle1.transfer(inv, spec, S, D, world, {pid}, dists=(sd, dd))
        else:
            dw, dbf = oracle1.redundant_backup(inv, spec, S, D, world, backup, {pid}, dist=dd), {}
        t2 = time.perf_counter()
        nb = sum((i.rng[1] - i.rng[0]) * 12 for infos in dw.values() for i in infos.values())
        nb += sum(x.size * 2 for x in dbf.values())
        copy_t += t1 - t0
        total_t += t2 - t1
        total_b += nb
        if p["layer"] == 0:
            l0_t += t2 - t1
            l0_b += nb
        n_params += 1
        n_elems += model.numel(p["shape"])
        del world, dw, dbf
    return {"value": round(total_b / total_t / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"the whole switch: all {n_params} parameters ({n_elems} elements), one parameter at a "
                      f"time, {total_b / 1e9:.1f} GB payload in {total_t:.1f} s; torch CPU threads={cores}",
            "full_switch_ms": round(total_t * 1e3, 1), "input_copy_s": round(copy_t, 1),
            "layer0_gbps": round(l0_b / l0_t / 1e9, 3) if l0_t else None,
            "nproc": os.cpu_count(), "cpu_model": _cpu_model()}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    args = parse()
    ws = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or ws != 1:
        print("bench.py measures one GPU: the reshard is simulated for every rank on a single device; "
              "run it with --gpus 1 (the benchmark has no multi-GPU mode).", file=sys.stderr)
        return 2

    import torch

    from elasticmegatron_amd import _native
    from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy
    from elasticmegatron_amd.megatron_manager.training_state import TrainingState
    from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
    from elasticmegatron_amd.transfer.transfer import TransferManager

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _native.load()
    _native.set_tuning(args.blocks_per_cu, bool(args.nontemporal), args.xcd_remap, args.run,
                       bool(args.persistent), args.lanes, args.units, chunk_index=bool(args.chunk_index),
                       warm_tables=bool(args.warm_tables))
    stream = torch.cuda.current_stream(dev)

    if args.copy_calibration_gib > 0:
        return copy_calibration(args, dev, stream)

    desc, spec_fn, src, dst, *opt = workloads()[args.workload]
    if args.share_rank is not None:
        return bench_share(args, desc, spec_fn, src, dst, dev, stream)
    if not args.low_memory and not args.ipc and not fits_twice(spec_fn(), dev):
        print(f"bench.py: two whole states of {args.workload} do not fit on this GPU; time one destination rank's "
              "share (--share-rank G) or a staged switch (--low-memory)", file=sys.stderr)
        return 2
    if args.low_memory and args.ipc:
        return bench_ipc_staged(args, desc, spec_fn, src, dst, dev)
    if args.low_memory:
        return bench_low_memory(args, desc, spec_fn, src, dst, dev)
    if args.megatron_buffers:
        return bench_megatron_buffers(args, desc, spec_fn, src, dst, dev, stream)
    if args.ipc:
        return bench_ipc(args, desc, spec_fn, src, dst, dev, stream)
    if args.adopt:
        return bench_adopt(args, desc, spec_fn, src, dst, dev, stream)
    if args.lost_ranks:
        return bench_lost_ranks(args, desc, spec_fn, src, dst, dev, stream)
    repad = bool(opt and opt[0])
    backup = ParallelStrategy.is_redundant_backup(src, dst)
    spec = spec_fn()
    t0 = time.time()
    if repad:
        ls = build_virtual_model(spec.with_padded_vocab(spec.padded_vocab_for_tp(
            src.tensor_model_parallel_size))).layout(src)
        ld = build_virtual_model(spec.with_padded_vocab(spec.padded_vocab_for_tp(
            dst.tensor_model_parallel_size))).layout(dst)
    else:
        space = build_virtual_model(spec)
        ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager(bf16_source=args.bf16_source)
    kind = "transfer" if backup is None else ("backup_up" if backup else "backup_down")
    plan = tm.compile(ls, ld, kind)
    tplan = tm.compile_tensors(ls, ld, kind) if args.tensors else None
    t_plan = time.time() - t0
    a = TrainingState.allocate(ls, dev)
    b = TrainingState.allocate(ld, dev, param=a.param if backup is not None else None)
    a.fill_synthetic(SEED, bf16=True)
    torch.cuda.synchronize()
    if args.shape_sweep is not None:
        return shape_sweep(args, desc, tm, plan, a, b, backup, ls.space.spec.padded_vocab_size if repad else None,
                           stream)
    if args.rank_shares:
        return rank_shares(args, desc, tm, plan, ls, ld, kind, a, b, backup,
                           ls.space.spec.padded_vocab_size if repad else None, stream)
    views = {}

    def step(a, b):
        if tplan is None:
            tm.execute(plan, a, b, stream)
            return
        if views.get("a") is not a or views.get("b") is not b:
            # One tensor view per buffer, as a caller holding per-tensor state passes them.  The cache
            # holds the states it was built from and is cleared before either is released.
            views.clear()
            views.update(a=a, b=b, v=(tplan.src.views(a), tplan.dst.views(b)))
        tm.execute_tensors(tplan, *views["v"], stream)

    print(f"[bench] {args.workload}: plan {plan.segments.shape[0]} segments, payload {plan.payload_bytes / 1e9:.2f} GB,"
          f" planning {t_plan:.2f}s", file=sys.stderr, flush=True)

    def check_destination():
        """Every destination element against the generator; None when --no-verify."""
        if args.no_verify:
            return None
        vocab_rows = ls.space.spec.padded_vocab_size if repad else None
        bad, first = b.verify_synthetic(SEED, bf16=backup is None, vocab_rows=vocab_rows)
        if bad:
            print(f"[bench] verification FAILED: {bad} elements, first {first}", file=sys.stderr)
        return bad == 0

    for _ in range(args.warmup):
        step(a, b)
    torch.cuda.synchronize()

    events = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    events[0].record(stream)
    for i in range(args.steps):
        step(a, b)
        events[i + 1].record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t_wall) * 1e3
    # Every step rewrites the whole destination with the same values, so the check after the last
    # timed step covers them all; run between the warm-up and the timed steps, its own pass over
    # the destination would leave the first timed launch cold.
    verified = check_destination()
    if verified is False:
        return 3
    step_ms = [events[i].elapsed_time(events[i + 1]) for i in range(args.steps)]
    flush = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device=dev)
    cold_ms = cold_launch_ms(lambda: step(a, b), flush, stream, 3)
    del flush
    ms = sum(step_ms) / len(step_ms)
    payload = plan.payload_bytes
    gbps = payload / (ms / 1e3) / 1e9
    traffic_gbps = plan.traffic_bytes / (ms / 1e3) / 1e9

    traffic = committed_traffic(args.workload, tm.bf16_source if backup is None else None, plan.traffic_bytes)

    out = {
        "metric": metric_for(args.workload, desc),
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16+fp32 (bitwise copy)",
        "data": "synthetic (seeded; bf16 ~N(0,0.02), main = upcast, exp_avg ~N(0,1e-3), exp_avg_sq = |N(0,1e-6)|)",
        "config": {"workload": desc, "params": spec.num_params(), "payload_bytes": payload,
                   "buffers": (f"one per stored tensor: {len(tplan.src)} source, {len(tplan.dst)} destination"
                               if tplan is not None else "four arenas per side"),
                   "read_bytes": plan.read_bytes, "bf16_source": tm.bf16_source if backup is None else None,
                   "segments": int((tplan or plan).segments.shape[0]), "verified_bit_exact": verified,
                   "wall_ms_per_step": round(wall_ms / args.steps, 4),
                   "min_ms": round(min(step_ms), 4), "max_ms": round(max(step_ms), 4),
                   "median_ms": round(sorted(step_ms)[len(step_ms) // 2], 4),
                   "first_third_ms": round(sum(step_ms[:max(1, len(step_ms) // 3)]) / max(1, len(step_ms) // 3), 4),
                   "last_third_ms": round(sum(step_ms[-max(1, len(step_ms) // 3):]) / max(1, len(step_ms) // 3), 4),
                   "launch": launch_shape(),
                   "cold_launch_ms": round(cold_ms, 4),
                   "reference_perf_line": {
                       "what": "the figures of the reference's perf log line (elastic_manager.py:158-178): GiB "
                               "of fp32 state the busiest rank would exchange with other ranks, per second of "
                               "this launch; a different quantity from value and roofline",
                       "communication_gib": round(plan.reference_comm_bytes / 2 ** 30, 3),
                       "gib_per_s": round(plan.reference_comm_bytes / 2 ** 30 / (ms / 1e3), 1)}},
        "roofline": {"bound": "hbm", "achieved": round(traffic_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(traffic_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic},
    }
    if tplan is not None:
        # The arena plan on the same allocations in this process, alternating with the per-tensor
        # plan, so that the two compare without the spread of placements between processes.
        out["config"]["same_process_ms"] = alternate_rounds(
            {"tensors": lambda: step(a, b), "arenas": lambda: tm.execute(plan, a, b, stream)}, stream)
    if args.placement_trials:
        import gc

        trials = []
        for _ in range(args.placement_trials):
            views.clear()
            del b
            gc.collect()
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
            b = TrainingState.allocate(ld, dev, param=a.param if backup is not None else None)
            for _ in range(2):
                step(a, b)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(5):
                step(a, b)
            e1.record(stream)
            torch.cuda.synchronize()
            trials.append(round(e0.elapsed_time(e1) / 5, 3))
        out["config"]["placement_trials_ms"] = trials
    if not args.no_verify:
        # The plan's own check of the destination against the source (emrs_plan_compare), timed
        # on its second call, when its grouped plan is built and cached.
        tm.verify(a, b, kind)
        torch.cuda.synchronize()
        t_v = time.perf_counter()
        report = tm.verify(a, b, kind)
        v_ms = (time.perf_counter() - t_v) * 1e3
        r_ms, r_bytes = read_ceiling(a, b, backup is None, stream)
        out["config"]["plan_verification"] = {
            "bit_exact": report.bit_exact, "elements": report.elements, "wall_ms": round(v_ms, 3),
            "read_ceiling_ms": round(r_ms, 3), "read_ceiling_bytes": r_bytes}
        if not report.bit_exact:
            print(f"[bench] plan verification FAILED: {report.lines()[:3]}", file=sys.stderr)
            return 3
    if not args.no_copy_ceiling:
        out["config"]["copy_ceiling"] = copy_ceiling(a, b, stream, traffic_gbps, plan.read_bytes, payload)
    views.clear()
    del b
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline: Oracle-1 over every parameter", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(spec, ls, src, dst, backup, a)
    if not args.no_e2e:
        a, out["config"]["reshard_e2e"] = reshard_end_to_end(a, spec, src, dst, repad, tm, args.no_verify)
    del a
    torch.cuda.empty_cache()
    print(json.dumps(out), flush=True)
    return 0


def committed_traffic(workload: str, bf16_source, algorithmic_bytes: int):
    """HBM bytes per launch from the committed PMC summary of ``workload`` (profiles/), or None when
    there is none for this bf16 source (None: fp32-only Group-ZeRO plans) or it was measured on a
    plan with other algorithmic bytes."""
    tf = os.path.join(ROOT, "profiles", f"{workload}.traffic.json")
    if not os.path.exists(tf):
        return None
    with open(tf) as f:
        rec = json.load(f)
    if rec.get("bf16_source", "cast") != bf16_source or rec.get("algorithmic_bytes_per_launch") != algorithmic_bytes:
        return None
    return rec.get("hbm_bytes_per_launch")


def bench_low_memory(args, desc, spec_fn, src, dst, dev):
    """Staged switches through the manager, alternating src -> dst -> src ...  A step is one whole
    switch: per optimizer kind, the destination arena's allocation, its launch and the release of
    the source arena (the source state of the next step is the destination of this one)."""
    import logging

    import torch

    from elasticmegatron_amd import ElasticMegatronManager

    quiet = logging.getLogger("bench.reshard")
    quiet.addHandler(logging.NullHandler())
    quiet.propagate = False
    spec = spec_fn()
    share = args.ipc_granule_bytes if args.shared_states else None
    mgr = ElasticMegatronManager([src, dst], spec, device=dev, low_memory=True, share_granule_bytes=share)
    lay = {s: mgr.space_for(s).layout(s) for s in (src, dst)}
    plans = {(a, b): mgr.transfer_manager.compile(lay[a], lay[b]) for a, b in ((src, dst), (dst, src))}
    mgr.training_state.fill_synthetic(SEED)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    order = [dst, src]
    cur = src
    for i in range(args.warmup):
        mgr.reshard(order[i % 2], logger=quiet)
        cur = order[i % 2]
    wall, launch, payload, traffic, stages = [], [], [], [], None
    for i in range(args.steps):
        nxt = dst if cur == src else src
        torch.cuda.synchronize()
        t = time.perf_counter()
        mgr.reshard(nxt, logger=quiet)
        torch.cuda.synchronize()
        wall.append((time.perf_counter() - t) * 1e3)
        stages = mgr.last_stage_ms
        launch.append(sum(s["execute"] for s in stages))
        p = plans[(cur, nxt)]
        payload.append(p.payload_bytes)
        traffic.append(p.traffic_bytes)
        cur = nxt
    bad = None
    if not args.no_verify:
        bad, first = mgr.training_state.verify_synthetic(SEED)
        if bad:
            print(f"[bench] verification FAILED: {bad} elements, first {first}", file=sys.stderr)
            return 3
    peak = torch.cuda.max_memory_allocated(dev)
    ms = sum(wall) / len(wall)
    launch_ms = sum(launch) / len(launch)
    gbps = sum(payload) / (sum(wall) / 1e3) / 1e9
    kern = sum(traffic) / (sum(launch) / 1e3) / 1e9
    la, lb = lay[src], lay[dst]
    both = sum(3 * x.fp32_numel * 4 + x.bf16_numel * 2 for x in (la, lb))
    out = {
        "metric": metric_for(args.workload, desc), "value": round(gbps, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16+fp32 (bitwise copy)",
        "data": "synthetic (seeded; bf16 ~N(0,0.02), main = upcast, exp_avg ~N(0,1e-3), exp_avg_sq = |N(0,1e-6)|)",
        "config": {"workload": desc + ", staged: one optimizer kind per launch, arenas allocated and released as it goes"
                   + (f", states in {share}-byte granules" if share else ""),
                   "params": spec.num_params(), "payload_bytes_per_switch": int(sum(payload) / len(payload)),
                   "launch_ms_per_switch": round(launch_ms, 4), "last_switch_stages_ms": stages,
                   "peak_allocated_bytes": int(peak), "both_whole_states_bytes": int(both),
                   "device_bytes": int(torch.cuda.get_device_properties(dev).total_memory),
                   "verified_bit_exact": None if bad is None else bad == 0,
                   "step": "one whole switch through ElasticMegatronManager.reshard, directions alternating"},
        "roofline": {"bound": "hbm", "achieved": round(kern, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(kern / HBM_PEAK_GBPS, 4), "traffic": None,
                     "note": "algorithmic bytes over the launches' time, allocation and release excluded"},
    }
    print(json.dumps(out), flush=True)
    return 0


def bench_megatron_buffers(args, desc, spec_fn, src, dst, dev, stream):
    """The switch on Megatron-shaped flat buffers (MegatronBuffers): every buffer a separate
    allocation, the per-tensor plan run on views of them.  The source buffers are filled and the
    destination checked on the device, piece by piece, with the seeded generator."""
    import torch

    from elasticmegatron_amd import _native
    from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy
    from elasticmegatron_amd.resharding.megatron_buffers import MegatronBuffers
    from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
    from elasticmegatron_amd.transfer.transfer import TransferManager

    spec = spec_fn()
    backup = ParallelStrategy.is_redundant_backup(src, dst)
    kind = "transfer" if backup is None else ("backup_up" if backup else "backup_down")
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager(bf16_source=args.bf16_source)
    arena_plan = tm.compile(ls, ld, kind)
    plan = tm.compile_tensors(ls, ld, kind)
    ms_, md = MegatronBuffers(ls), MegatronBuffers(ld)
    sbuf, dbuf = ms_.allocate(dev), md.allocate(dev)
    if backup is not None:  # the model shards do not change under Group ZeRO: one bf16 buffer set
        for key in list(dbuf):
            if key[0] == "param":
                dbuf[key] = sbuf[key]
    s_ptrs, d_ptrs = [sbuf[k].data_ptr() for k in ms_.keys()], [dbuf[k].data_ptr() for k in md.keys()]
    _native.synth_fill(ms_.remap_pieces(ls.pieces()), s_ptrs, ms_.byte_sizes(), SEED, stream.cuda_stream)
    src_views, dst_views = ms_.tensor_views(plan.src, sbuf), md.tensor_views(plan.dst, dbuf)
    torch.cuda.synchronize()
    print(f"[bench] {args.workload} on Megatron buffers: {len(ms_.specs)} source and {len(md.specs)} destination "
          f"buffers, {len(plan.src)} / {len(plan.dst)} tensors, {plan.segments.shape[0]} segments",
          file=sys.stderr, flush=True)
    def check_destination():
        """Every destination element against the generator; None when --no-verify."""
        if args.no_verify:
            return None
        bad, _ = _native.synth_verify(md.remap_pieces(ld.pieces(include_bf16=backup is None)), d_ptrs,
                                      md.byte_sizes(), SEED, stream.cuda_stream)
        if bad:
            print(f"[bench] verification FAILED: {bad} elements", file=sys.stderr)
        return bad == 0

    for _ in range(args.warmup):
        tm.execute_tensors(plan, src_views, dst_views, stream)
    torch.cuda.synchronize()
    events = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    events[0].record(stream)
    for i in range(args.steps):
        tm.execute_tensors(plan, src_views, dst_views, stream)
        events[i + 1].record(stream)
    torch.cuda.synchronize()
    verified = check_destination()  # after the timed steps, as in the arena benchmark
    if verified is False:
        return 3
    step_ms = [events[i].elapsed_time(events[i + 1]) for i in range(args.steps)]
    ms = sum(step_ms) / len(step_ms)
    traffic_gbps = arena_plan.traffic_bytes / (ms / 1e3) / 1e9
    out = {
        "metric": metric_for(args.workload, desc), "value": round(plan.payload_bytes / (ms / 1e3) / 1e9, 2),
        "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16+fp32 (bitwise copy)",
        "data": "synthetic (seeded; bf16 ~N(0,0.02), main = upcast, exp_avg ~N(0,1e-3), exp_avg_sq = |N(0,1e-6)|)",
        "config": {"workload": desc + ", on Megatron-shaped flat buffers (one allocation each, padding in place)",
                   "params": spec.num_params(), "payload_bytes": plan.payload_bytes,
                   "buffers": f"{len(ms_.specs)} source, {len(md.specs)} destination flat buffers; "
                              f"{len(plan.src)} / {len(plan.dst)} tensor views",
                   "segments": int(plan.segments.shape[0]), "verified_bit_exact": verified,
                   "min_ms": round(min(step_ms), 4), "max_ms": round(max(step_ms), 4), "launch": launch_shape()},
        "roofline": {"bound": "hbm", "achieved": round(traffic_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(traffic_gbps / HBM_PEAK_GBPS, 4), "traffic": None},
    }
    print(json.dumps(out), flush=True)
    return 0


def bench_ipc(args, desc, spec_fn, src, dst, dev, stream):
    """The switch from another process's exported state (the reference's inter-process hand-off,
    ipc_manager.py:54-155): a child process allocates the source in granules, fills it and sends
    the payload; this process maps the granules and times the switch from them into its own
    arenas.  The mappings are closed before the child is told to exit."""
    import torch

    from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy
    from elasticmegatron_amd.megatron_manager.training_state import TrainingState
    from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
    from elasticmegatron_amd.transfer import ipc_manager as ipc
    from elasticmegatron_amd.transfer.transfer import TransferManager, backup_kind

    # A Group-ZeRO switch copies the bf16 params here: the exporter frees its memory.
    backup = ParallelStrategy.is_redundant_backup(src, dst)
    kind = "transfer" if backup is None else backup_kind(backup, copy_bf16=True)
    if backup is not None:
        desc = desc.replace(", fp32 only", "") + ", fp32 and the bf16 params copied"
    spec = spec_fn()
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    child = spawn_exporter(spec, src, args.ipc_granule_bytes)
    state = None
    try:
        tm = TransferManager(bf16_source=args.bf16_source)
        plan = tm.compile_granules(ls, ld, args.ipc_granule_bytes, None, kind)
        arena_plan = tm.compile(ls, ld, kind)
        b = TrainingState.allocate(ld, dev)
        line = exporter_payload(child)
        if line is None:
            return 1
        state, _ = ipc.receive_training_state(line, dev, space=space)
        print(f"[bench] {args.workload}: {len(state.buffers)} granules mapped, {plan.segments.shape[0]} segments",
              file=sys.stderr, flush=True)
        tm.prepare(plan, dev)
        for _ in range(args.warmup):
            tm.execute_states(plan, state, b, stream)
        torch.cuda.synchronize()
        events = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
        events[0].record(stream)
        for i in range(args.steps):
            tm.execute_states(plan, state, b, stream)
            events[i + 1].record(stream)
        torch.cuda.synchronize()
        verified = None
        if not args.no_verify:
            bad, first = b.verify_synthetic(SEED)
            report = tm.verify(state, b, kind)
            verified = bad == 0 and report.bit_exact
            if not verified:
                print(f"[bench] verification FAILED: {bad} elements, first {first}; "
                      f"{report.lines()[:3]}", file=sys.stderr)
                return 3
        n_granules = len(state.buffers)
        owned = mapped_vs_owned(args, tm, plan, ls, state, b, dev, stream)
        if owned.get("verified_bit_exact") is False:
            return 3
    finally:
        end_exporter(child, state)
    step_ms = [events[i].elapsed_time(events[i + 1]) for i in range(args.steps)]
    ms = sum(step_ms) / len(step_ms)
    traffic_gbps = arena_plan.traffic_bytes / (ms / 1e3) / 1e9
    out = {
        "metric": metric_for(args.workload, desc), "value": round(plan.payload_bytes / (ms / 1e3) / 1e9, 2),
        "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16+fp32 (bitwise copy)",
        "data": "synthetic (seeded; bf16 ~N(0,0.02), main = upcast, exp_avg ~N(0,1e-3), exp_avg_sq = |N(0,1e-6)|)",
        "config": {"workload": desc + f", from another process's state in {args.ipc_granule_bytes}-byte granules",
                   "params": spec.num_params(), "payload_bytes": plan.payload_bytes, "granules": n_granules,
                   "segments": int(plan.segments.shape[0]), "verified_bit_exact": verified,
                   "exporter_exit_status": child.returncode, "mapped_vs_owned": owned,
                   "min_ms": round(min(step_ms), 4), "max_ms": round(max(step_ms), 4), "launch": launch_shape()},
        "roofline": {"bound": "hbm", "achieved": round(traffic_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(traffic_gbps / HBM_PEAK_GBPS, 4), "traffic": None},
    }
    print(json.dumps(out), flush=True)
    return 0


def timed_launches(run, steps, warmup, stream):
    """ms of each of ``steps`` launches of ``run`` after ``warmup`` untimed ones (events on
    ``stream``, the launches' own stream)."""
    import torch

    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    events = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    events[0].record(stream)
    for i in range(steps):
        run()
        events[i + 1].record(stream)
    torch.cuda.synchronize()
    return [events[i].elapsed_time(events[i + 1]) for i in range(steps)]


def bench_adopt(args, desc, spec_fn, src, dst, dev, stream):
    """A Group-ZeRO switch between shared states this process owns: the new state either gets
    instance 0 copied into granules of its own, or takes over the old state's leading granules
    (all of instance 0) and the plan writes only the other instances.  Both launches are timed on
    the same source, one after the other (two new states do not fit beside the source), each
    checked against the generator; then ElasticMegatronManager.reshard runs end to end both ways
    (without release_source the old state is kept whole, so nothing is taken over).  Every new
    state's granules come from torch's cache, as in a running job: memory handed back to the driver
    is cleared before it is handed out again, at tens of GB/s, which would swamp the comparison."""
    import gc

    import torch

    from elasticmegatron_amd import ElasticMegatronManager
    from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy
    from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
    from elasticmegatron_amd.transfer.ipc_manager import SharedTrainingState
    from elasticmegatron_amd.transfer.transfer import TransferManager, adoptable_granules, backup_kind

    backup = ParallelStrategy.is_redundant_backup(src, dst)
    if backup is None:
        print("--adopt times a Group-ZeRO workload", file=sys.stderr)
        return 2
    g, kind = args.ipc_granule_bytes, backup_kind(backup)
    spec = spec_fn()
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    n = adoptable_granules(ls, ld, g, kind)
    tm = TransferManager(bf16_source=args.bf16_source)
    plans = {"copied": tm.compile_granules(ls, ld, g, g, kind), "taken_over": tm.compile_granules(ls, ld, g, g, kind,
                                                                                                  adopt_granules=n)}
    a = SharedTrainingState.allocate(ls, dev, g)
    a.fill_synthetic(SEED)
    param = [a.tensors[x] for x in a.buffers.granules_of(3)]
    res = {}
    for name, plan in plans.items():
        before = torch.cuda.memory_allocated(dev)
        b = SharedTrainingState.allocate(ld, dev, g, param_granules=param,
                                         adopted=a.leading_fp32_granules(n) if name == "taken_over" else None)
        new_bytes = torch.cuda.memory_allocated(dev) - before
        both_states = torch.cuda.memory_allocated(dev)        # source and new state together
        tm.prepare(plan, dev)
        step_ms = timed_launches(lambda: tm.execute_states(plan, a, b, stream), args.steps, args.warmup, stream)
        bad, first = b.verify_synthetic(SEED)
        exact = bad == 0 and tm.verify(a, b, kind).bit_exact
        if not exact:
            print(f"[bench] {name}: verification FAILED: {bad} elements, first {first}", file=sys.stderr)
            return 3
        ms = sum(step_ms) / len(step_ms)
        res[name] = {"ms": round(ms, 3), "min_ms": round(min(step_ms), 3), "payload_bytes": plan.payload_bytes,
                     "traffic_bytes": plan.traffic_bytes, "new_state_allocated_bytes": new_bytes,
                     "both_states_allocated_bytes": both_states,
                     "traffic_gbps": round(plan.traffic_bytes / ms / 1e6, 1),
                     "verified_bit_exact": exact}
        print(f"[bench] {name}: {ms:.2f} ms, {res[name]['traffic_gbps']} GB/s", file=sys.stderr, flush=True)
        del b
        gc.collect()      # the granules stay in torch's cache for the next state

    def manager_switch(release):
        mgr = ElasticMegatronManager([src, dst], spec, device=dev, training_state=a, share_granule_bytes=g,
                                     release_source=release)
        mgr.reshard(dst, is_meta_device=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        new = mgr.reshard(dst, logger=logging.getLogger("bench"))     # keeps stdout to the JSON line
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3
        bad, _ = new.verify_synthetic(SEED)
        return new, {"wall_ms": round(wall, 2), "launch_ms": round(mgr.last_transfer_ms, 2),
                     "verified_bit_exact": bad == 0}

    kept, e2e_copy = manager_switch(False)
    del kept
    gc.collect()
    _, e2e_adopt = manager_switch(True)         # releases the source: last
    if not (e2e_copy["verified_bit_exact"] and e2e_adopt["verified_bit_exact"]):
        print("[bench] a manager switch FAILED verification", file=sys.stderr)
        return 3
    res["copied"]["reshard_end_to_end"], res["taken_over"]["reshard_end_to_end"] = e2e_copy, e2e_adopt
    t = res["taken_over"]
    out = {
        "metric": f"Group-ZeRO switch between shared states, instance 0 taken over: ms per launch, {desc}, 1 GPU",
        "value": t["ms"], "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": t["ms"], "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 (bitwise copy)", "data": "synthetic (seeded)",
        "config": {"workload": desc + f", both states in {g}-byte granules", "params": spec.num_params(),
                   "granules_taken_over_per_fp32_arena": n,
                   "speedup_vs_copied": round(res["copied"]["ms"] / t["ms"], 3),
                   **res, "launch": launch_shape()},
        "roofline": {"bound": "hbm", "achieved": t["traffic_gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(t["traffic_gbps"] / HBM_PEAK_GBPS, 4),
                     "traffic": committed_traffic(f"{args.workload}.taken_over", None, t["traffic_bytes"])},
    }
    print(json.dumps(out), flush=True)
    return 0


def bench_lost_ranks(args, desc, spec_fn, src, dst, dev, stream):
    """A Group-ZeRO switch timed twice on the same arenas: plain, then with the ``--lost-ranks``
    source ranks' fp32 state poisoned with NaN and each of their shards read from another
    optimizer instance.  Both results are checked against the generator, the second also by the
    plan's comparison against the copies it read."""
    import torch

    from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy
    from elasticmegatron_amd.megatron_manager.training_state import TrainingState
    from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
    from elasticmegatron_amd.transfer.transfer import TransferManager, backup_kind

    backup = ParallelStrategy.is_redundant_backup(src, dst)
    if backup is None:
        print("--lost-ranks times a Group-ZeRO workload: other switches have no second copy to read", file=sys.stderr)
        return 2
    kind, lost = backup_kind(backup), args.lost_ranks
    spec = spec_fn()
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager(bf16_source=args.bf16_source)
    plans = {"plain": tm.compile(ls, ld, kind), "lost": tm.compile(ls, ld, kind, lost_ranks=lost)}
    a = TrainingState.allocate(ls, dev)
    a.fill_synthetic(SEED)
    b = TrainingState.allocate(ld, dev, param=a.param)
    res = {}
    for name, plan in plans.items():
        if name == "lost":
            for g in lost:
                lo, hi = ls.rank_fp32_slice(g)
                for t in (a.main, a.exp_avg, a.exp_avg_sq):
                    t[lo:hi].fill_(float("nan"))
        for t in (b.main, b.exp_avg, b.exp_avg_sq):
            t.fill_(float("nan"))
        tm.prepare(plan, dev)
        step_ms = timed_launches(lambda: tm.execute(plan, a, b, stream), args.steps, args.warmup, stream)
        bad, first = b.verify_synthetic(SEED, bf16=False)
        exact = bad == 0 and tm.verify(a, b, kind, lost_ranks=lost if name == "lost" else ()).bit_exact
        if not exact:
            print(f"[bench] {name}: verification FAILED: {bad} elements, first {first}", file=sys.stderr)
            return 3
        ms = sum(step_ms) / len(step_ms)
        res[name] = {"ms": round(ms, 3), "min_ms": round(min(step_ms), 3), "traffic_bytes": plan.traffic_bytes,
                     "traffic_gbps": round(plan.traffic_bytes / ms / 1e6, 1), "verified_bit_exact": exact}
        print(f"[bench] {name}: {ms:.2f} ms", file=sys.stderr, flush=True)
    t = res["lost"]
    out = {
        "metric": f"Group-ZeRO switch with lost ranks read from another instance: ms per launch, {desc}, 1 GPU",
        "value": t["ms"], "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": t["ms"], "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 (bitwise copy)", "data": "synthetic (seeded); the lost ranks' fp32 state poisoned with NaN",
        "config": {"workload": desc, "params": spec.num_params(), "lost_ranks": list(lost), **res,
                   "launch": launch_shape()},
        "roofline": {"bound": "hbm", "achieved": t["traffic_gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(t["traffic_gbps"] / HBM_PEAK_GBPS, 4), "traffic": None},
    }
    print(json.dumps(out), flush=True)
    return 0


def spawn_exporter(spec, strategy, granule_bytes):
    """The exporting process of a hand-off: a child that allocates the state of ``strategy`` in
    granules, fills it with the seeded values and sends the payload on its stdout."""
    import dataclasses
    import subprocess

    from elasticmegatron_amd.transfer import ipc_manager as ipc

    return subprocess.Popen(
        [sys.executable, "-m", "elasticmegatron_amd.transfer.ipc_export", "--model-spec",
         json.dumps(dataclasses.asdict(spec)), "--strategy", json.dumps(ipc.strategy_to_dict(strategy)), "--seed",
         str(SEED), "--granule-bytes", str(granule_bytes)],
        cwd=ROOT, stdin=subprocess.PIPE, stdout=subprocess.PIPE, text=True)


def exporter_payload(child, timeout_s=600):
    """The payload line the exporter sends, or None (reported) when it sends nothing."""
    import select

    if not select.select([child.stdout], [], [], timeout_s)[0]:
        print(f"bench.py --ipc: the exporting process sent nothing in {timeout_s} s", file=sys.stderr)
        return None
    line = child.stdout.readline()
    if not line:
        print(f"bench.py --ipc: the exporting process exited with {child.wait()}", file=sys.stderr)
        return None
    return line


def end_exporter(child, state):
    """Close what is still mapped, then tell the exporter to free its memory and wait for it."""
    import subprocess

    from elasticmegatron_amd.transfer import ipc_manager as ipc

    if state is not None:
        state.close()
    if child.poll() is None:
        try:
            ipc.notify_release(child.stdin)
            child.stdin.close()
        except BrokenPipeError:
            pass
        try:
            child.wait(timeout=120)
        except subprocess.TimeoutExpired:
            child.kill()
            child.wait()


def bench_ipc_staged(args, desc, spec_fn, src, dst, dev):
    """A staged switch (ElasticMegatronManager(low_memory=True)) from another process's state: after
    each optimizer kind's launch the source arena's mappings are closed and the exporter frees it
    before the next kind's destination arena is allocated, so the device holds the source, the
    destination's bf16 params and one fp32 arena at most.  The switch consumes its source, so one
    switch is timed per run, its plans prepared on the meta-device pass beforehand."""
    import logging

    import torch

    from elasticmegatron_amd import ElasticMegatronManager
    from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy
    from elasticmegatron_amd.transfer import ipc_manager as ipc
    from elasticmegatron_amd.transfer.transfer import backup_kind

    quiet = logging.getLogger("bench.reshard")
    quiet.addHandler(logging.NullHandler())
    quiet.propagate = False
    spec = spec_fn()
    mgr = ElasticMegatronManager([src, dst], spec, device="meta", low_memory=True)
    child = spawn_exporter(spec, src, args.ipc_granule_bytes)
    state, free_before_release = None, []
    try:
        line = exporter_payload(child)
        if line is None:
            return 1
        state, _ = ipc.receive_training_state(line, dev, space=mgr.virtual_param_space)
        hook = ipc.release_hook(child.stdin, child.stdout)

        def on_release(kind):
            free_before_release.append(torch.cuda.mem_get_info(dev)[0])
            hook(kind)

        state.on_release = on_release
        n_granules = len(state.buffers)
        mgr.attach_training_state(state)
        mgr.reshard(dst, is_meta_device=True)
        # A received state cannot keep its bf16 params: a Group-ZeRO switch copies them.
        backup = ParallelStrategy.is_redundant_backup(src, dst)
        kind = "transfer" if backup is None else backup_kind(backup, copy_bf16=True)
        plans = mgr.transfer_manager.staged_for_states(state.layout, mgr.space_for(dst).layout(dst),
                                                       state.granule_bytes, None, kind)
        torch.cuda.synchronize()
        t = time.perf_counter()
        new = mgr.reshard(dst, logger=quiet)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t) * 1e3
        state = None
        stages = mgr.last_stage_ms
        bad = None
        if not args.no_verify:
            bad, first = new.verify_synthetic(SEED)
            if bad:
                print(f"[bench] verification FAILED: {bad} elements, first {first}", file=sys.stderr)
                return 3
        peak_here = torch.cuda.max_memory_allocated(dev)
    finally:
        end_exporter(child, state)
    total = torch.cuda.get_device_properties(dev).total_memory
    payload = sum(p.payload_bytes for p in plans)
    traffic = sum(p.payload_bytes + p.read_bytes for p in plans)
    launch_ms = sum(s["execute"] for s in stages)
    kern = traffic / (launch_ms / 1e3) / 1e9
    ls = mgr.space_for(src).layout(src)
    src_bytes = 3 * ls.fp32_numel * 4 + ls.bf16_numel * 2
    out = {
        "metric": metric_for(args.workload, desc), "value": round(payload / (wall / 1e3) / 1e9, 2), "unit": "GB/s",
        "n_gpus": 1, "steps": 1, "warmup": 0, "ms_per_step": round(wall, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16+fp32 (bitwise copy)",
        "data": "synthetic (seeded; bf16 ~N(0,0.02), main = upcast, exp_avg ~N(0,1e-3), exp_avg_sq = |N(0,1e-6)|)",
        "config": {"workload": desc + f", from another process's state in {args.ipc_granule_bytes}-byte granules, "
                               "staged: one optimizer kind per launch, each source arena freed by the exporter "
                               "after its launch",
                   "params": spec.num_params(), "payload_bytes": payload, "granules": n_granules,
                   "launch_ms": round(launch_ms, 4), "stages_ms": stages,
                   "source_state_bytes": src_bytes, "peak_allocated_here_bytes": int(peak_here),
                   "device_used_before_each_release_bytes": [int(total - f) for f in free_before_release],
                   "device_bytes": int(total), "verified_bit_exact": None if bad is None else bad == 0,
                   "exporter_exit_status": child.returncode,
                   "step": "one whole switch through ElasticMegatronManager.reshard: per optimizer kind, the "
                           "destination arena's allocation, its launch, the close of the source arena's "
                           "mappings and the exporter's free of it"},
        "roofline": {"bound": "hbm", "achieved": round(kern, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(kern / HBM_PEAK_GBPS, 4), "traffic": None,
                     "note": "algorithmic bytes over the launches' time, allocation and release excluded"},
    }
    print(json.dumps(out), flush=True)
    return 0


def fits_twice(spec, dev) -> bool:
    """Whether two whole states of the model (14 bytes per parameter each) fit in the device's memory."""
    import torch

    return 2 * 14 * spec.num_params() < torch.cuda.get_device_properties(dev).total_memory * 0.97


def bench_share(args, desc, spec_fn, src, dst, dev, stream):
    """One destination rank's share of the switch (``TransferManager.compile_share_tensors``) on the
    tensors it touches alone, each allocated on its own as a Megatron job holds them: the rank's own
    optimizer tensors and its model shard's bf16 params, and the source tensors it reads.  With one
    rank per GPU this is GPU g's part of the switch at its real size; its reads of other ranks' tensors
    would come over xGMI.  Checked against the generator on every fp32 element the rank holds and, bit
    for bit, by the share's own comparison.  ``--share-rank -1`` runs every rank's share in turn and
    gives the switch's time with one rank per GPU as the slowest rank's, each rank taking the longer
    of its HBM time and its remote reads at the xGMI ingress rate."""
    import gc

    import torch

    from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
    from elasticmegatron_amd.transfer.transfer import TransferManager

    spec = spec_fn()
    space = build_virtual_model(spec)
    space.register_reshard(src, dst)
    ls, ld = space.layout(src), space.layout(dst)
    tm = TransferManager(bf16_source=args.bf16_source)
    common = {"steps": args.steps, "warmup": args.warmup, "n_gpus": 1, "higher_is_better": True, "scaling": "weak",
              "vs_baseline": None, "dtype": "bf16+fp32 (bitwise copy)",
              "data": "synthetic (seeded; bf16 ~N(0,0.02), main = upcast, exp_avg ~N(0,1e-3), "
                      "exp_avg_sq = |N(0,1e-6)|)"}
    if args.share_rank >= 0:
        row = share_run(args, tm, ls, ld, args.share_rank, dev, stream)
        if isinstance(row, int):
            return row
        g = args.share_rank
        out = {"metric": metric_for(args.workload, desc) + f", destination rank {g}'s share",
               "value": round(row["payload_bytes"] / (row["ms"] / 1e3) / 1e9, 2), "unit": "GB/s",
               "ms_per_step": row["ms"], **common,
               "config": {"workload": desc + f", destination rank {g}'s share on the tensors it touches",
                          "params": spec.num_params(), **row, "launch": launch_shape()},
               "roofline": {"bound": "hbm", "achieved": row["traffic_gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                            "frac": round(row["traffic_gbps"] / HBM_PEAK_GBPS, 4), "traffic": None}}
        print(json.dumps(out), flush=True)
        return 0
    rows = []
    for g in range(dst.world_size):
        row = share_run(args, tm, ls, ld, g, dev, stream)
        if isinstance(row, int):
            return row
        rows.append(row)
        gc.collect()
        torch.cuda.empty_cache()
    per_gpu = [max(r["ms"], r["remote_at_xgmi_ingress_ms"]) for r in rows]
    slowest = max(range(len(rows)), key=lambda i: per_gpu[i])
    payload = sum(r["payload_bytes"] for r in rows)
    out = {"metric": metric_for(args.workload, desc) + ", every destination rank's share",
           "value": round(payload / (per_gpu[slowest] / 1e3) / 1e9, 2), "unit": "GB/s",
           "ms_per_step": per_gpu[slowest], **common,
           "config": {"workload": desc + ", every destination rank's share on the tensors it touches, one after "
                                         "another on one GPU",
                      "params": spec.num_params(), "ranks": len(rows),
                      "what": "value and ms_per_step: the switch with one rank per GPU, bound by the slowest rank, "
                              "each rank taking the longer of its measured HBM time and its remote reads at "
                              f"{XGMI_INGRESS_GBPS:.0f} GB/s of xGMI ingress (projected, not measured on several GPUs)",
                      "slowest_rank": slowest, "max_hbm_ms": max(r["ms"] for r in rows),
                      "max_remote_xgmi_ms": max(r["remote_at_xgmi_ingress_ms"] for r in rows),
                      "min_traffic_gbps": min(r["traffic_gbps"] for r in rows),
                      "max_traffic_gbps": max(r["traffic_gbps"] for r in rows),
                      "verified_bit_exact": all(r["verified_bit_exact"] is not False for r in rows),
                      "launch": launch_shape(), "shares": rows}}
    print(json.dumps(out), flush=True)
    return 0


def share_run(args, tm, ls, ld, g, dev, stream):
    """Rank g's share on its own tensors: allocate, fill, time, check.  Returns its figures, or an
    exit code."""
    import numpy as np
    import torch

    from elasticmegatron_amd import _native
    from elasticmegatron_amd.resharding.layout import ARENA_PARAM
    from elasticmegatron_amd.resharding.shares import pull_bytes

    t0 = time.time()
    plan = tm.compile_share_tensors(ls, ld, g)
    planning_s = time.time() - t0
    sb, db = plan.src, plan.dst
    sizes = sum(sb.nbytes()[i] for i in plan.src_refs), sum(db.nbytes()[i] for i in plan.dst_refs)
    free = torch.cuda.mem_get_info(dev)[0]
    print(f"[bench] {args.workload} rank {g}: {len(plan.segments)} segments over {len(plan.src_refs)} source and "
          f"{len(plan.dst_refs)} destination tensors ({sizes[0] / 1e9:.1f} + {sizes[1] / 1e9:.1f} GB; "
          f"{free / 1e9:.1f} GB free); planning {planning_s:.1f} s", file=sys.stderr, flush=True)
    if sum(sizes) > free - (8 << 30):
        print("bench.py --share-rank: the share's tensors do not fit", file=sys.stderr)
        return 2

    def alloc(bufs, refs):
        out = [None] * len(bufs)
        for i in refs:
            out[i] = torch.empty(bufs.numel[i], device=dev,
                                 dtype=torch.bfloat16 if bufs.arena[i] == ARENA_PARAM else torch.float32)
        return out

    src_t, dst_t = alloc(sb, plan.src_refs), alloc(db, plan.dst_refs)

    def by_tensor(pieces, bufs, tensors):
        """The generator pieces of the allocated tensors, re-addressed by tensor, in batches of at most
        128 tensors: (pieces, pointers, bytes)."""
        ids = {}
        for p in pieces:
            b, loc = bufs.locate(int(p["buf"]), int(p["buf_off"]))
            if tensors[b] is not None:
                q = p.copy()
                q["buf_off"] = loc
                ids.setdefault(b, []).append(q)
        keys = sorted(ids)
        for lo in range(0, len(keys), 128):
            batch = keys[lo:lo + 128]
            rows = []
            for j, b in enumerate(batch):
                for q in ids[b]:
                    q["buf"] = j
                    rows.append(q)
            yield (np.array(rows, dtype=pieces.dtype), [tensors[b].data_ptr() for b in batch],
                   [tensors[b].numel() * tensors[b].element_size() for b in batch])

    for pcs, ptrs, nb in by_tensor(ls.pieces(), sb, src_t):
        _native.synth_fill(pcs, ptrs, nb, SEED, stream.cuda_stream)
    for _ in range(args.warmup):
        tm.execute_tensors(plan, src_t, dst_t, stream)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        tm.execute_tensors(plan, src_t, dst_t, stream)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    verified = None
    if not args.no_verify:
        bad = 0
        own = [t if t is not None and db.arena[i] != ARENA_PARAM else None for i, t in enumerate(dst_t)]
        for pcs, ptrs, nb in by_tensor(ld.pieces(include_bf16=False), db, own):
            n, _ = _native.synth_verify(pcs, ptrs, nb, SEED, stream.cuda_stream)
            bad += n
        stats = plan.native.compare([0 if t is None else t.data_ptr() for t in src_t],
                                    [0 if t is None else t.data_ptr() for t in dst_t], stream=stream.cuda_stream)
        verified = bad == 0 and int(stats["mismatches"].sum()) == 0
        if not verified:
            print(f"[bench] share of rank {g}: verification FAILED: {bad} generator mismatches, "
                  f"{int(stats['mismatches'].sum())} plan mismatches", file=sys.stderr)
            return 3
    per_rank, _ = tm.compile_shares(ls, ld)
    fp32, param = pull_bytes(per_rank[g].segments, ls)
    local = int(fp32[g]) if g < len(fp32) else 0
    remote = int(fp32.sum()) - local + param
    traffic = plan.payload_bytes + plan.read_bytes
    return {"rank": g, "ms": round(ms, 4), "segments": int(len(plan.segments)),
            "payload_bytes": plan.payload_bytes, "read_bytes": plan.read_bytes,
            "traffic_gbps": round(traffic / (ms / 1e3) / 1e9, 1),
            "source_tensors": len(plan.src_refs), "destination_tensors": len(plan.dst_refs),
            "source_tensor_bytes": sizes[0], "destination_tensor_bytes": sizes[1],
            "read_local_bytes": local, "read_remote_bytes": remote,
            "remote_at_xgmi_ingress_ms": round(remote / (XGMI_INGRESS_GBPS * 1e9) * 1e3, 3),
            "planning_s": round(planning_s, 2), "verified_bit_exact": verified}


def mapped_vs_owned(args, tm, plan, ls, mapped, b, dev, stream):
    """The granule plan from the mapped source and from a source of the same granules allocated in
    this process, taking turns on the same destination: what reading another process's memory
    costs, without the spread of placements between processes.  Skipped when the second source
    does not fit beside the first."""
    import gc

    import torch

    from elasticmegatron_amd.transfer.ipc_manager import SharedTrainingState

    need = sum(mapped.buffers.nbytes())
    free = torch.cuda.mem_get_info(dev)[0]
    if free < need + (4 << 30):
        return {"skipped": f"a second source of {need} bytes does not fit in {free} free bytes"}
    owned = SharedTrainingState.allocate(ls, dev, args.ipc_granule_bytes)
    try:
        owned.fill_synthetic(SEED)
        rounds = alternate_rounds({"mapped": lambda: tm.execute_states(plan, mapped, b, stream),
                                   "owned": lambda: tm.execute_states(plan, owned, b, stream)}, stream)
        rounds["verified_bit_exact"] = None if args.no_verify else b.verify_synthetic(SEED)[0] == 0
    finally:
        del owned
        gc.collect()
        torch.cuda.empty_cache()
    if rounds["verified_bit_exact"] is False:
        print("[bench] the switch from the owned source differs from the generator", file=sys.stderr)
    return rounds


def shape_sweep(args, desc, tm, plan, a, b, backup, vocab_rows, stream):
    """Each launch shape of --shape-sweep, timed on the same allocations in one process: round after
    round, every shape runs --warmup untimed and --steps timed launches.  Each shape's output is
    checked bit-exact once.  Physical placement moves all shapes together, so the shapes compare to
    within the spread between rounds."""
    import torch

    from elasticmegatron_amd import _native

    rows = [{"shape": shp or "default", "ms": [], "cold_ms": []} for shp in args.shape_sweep]
    flush = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device=a.main.device)
    try:
        for r in range(args.rounds):
            for shp, row in zip(args.shape_sweep, rows):
                try:
                    _native.set_tuning(**shp)
                except _native.EmrsError as e:
                    print(f"[bench] launch shape {shp}: {e}", file=sys.stderr)
                    return 2
                if r == 0:
                    row["launch"] = launch_shape()
                    for x in (b.main, b.exp_avg, b.exp_avg_sq):
                        x.fill_(float("nan"))
                    if backup is None:
                        b.param.zero_()
                    tm.execute(plan, a, b, stream)
                    torch.cuda.synchronize()
                    bad, first = b.verify_synthetic(SEED, bf16=backup is None, vocab_rows=vocab_rows)
                    if bad:
                        print(f"[bench] launch shape {shp}: verification FAILED: {bad} elements, first {first}",
                              file=sys.stderr)
                        return 3
                for _ in range(args.warmup):
                    tm.execute(plan, a, b, stream)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(args.steps):
                    tm.execute(plan, a, b, stream)
                e1.record(stream)
                torch.cuda.synchronize()
                row["ms"].append(round(e0.elapsed_time(e1) / args.steps, 4))
                row["cold_ms"].append(round(cold_launch_ms(lambda: tm.execute(plan, a, b, stream), flush, stream,
                                                           args.steps), 4))
    finally:
        _native.set_tuning()
    for row in rows:
        row["best_ms"] = min(row["ms"])
        row["best_cold_ms"] = min(row["cold_ms"])
        row["traffic_tbps_at_best"] = round(plan.traffic_bytes / (row["best_ms"] / 1e3) / 1e12, 3)
    print(json.dumps({"workload": desc, "what": "launch shapes on the same allocations in one process; ms: "
                      "back-to-back launches, cold_ms: each launch after a fill of other memory",
                      "steps": args.steps, "warmup": args.warmup, "rounds": args.rounds,
                      "traffic_bytes": plan.traffic_bytes, "verified_bit_exact": True, "shapes": rows}), flush=True)
    return 0


FLUSH_BYTES = 512 << 20  # more than the 256 MB memory-side cache


def cold_launch_ms(run, flush, stream, n):
    """Mean time of ``n`` launches of ``run``, each straight after a fill of ``flush`` (other memory,
    larger than the memory-side cache), as a single switch in a training job follows other kernels."""
    import torch

    total = 0.0
    for i in range(n):
        flush.fill_(i & 0xFF)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        run()
        e1.record(stream)
        torch.cuda.synchronize()
        total += e0.elapsed_time(e1)
    return total / n


XGMI_INGRESS_GBPS = 7 * 153.0  # seven peer links per MI355X, each about 153 GB/s one way


def rank_shares(args, desc, tm, plan, ls, ld, kind, a, b, backup, vocab_rows, stream):
    """Each destination rank's share of the plan (``TransferManager.compile_shares``), timed on its
    own after the whole plan, on the same allocations, with its reads split into the source rank of
    the same number (local with one rank per GPU) and the others (over xGMI then).  The destination
    is first overwritten, then written by the shares alone and checked against the generator."""
    import torch

    from elasticmegatron_amd.resharding.shares import pull_bytes

    per_rank, rest = tm.compile_shares(ls, ld, kind)
    arenas = [b.main, b.exp_avg, b.exp_avg_sq] + ([b.param] if backup is None else [])
    for t in arenas:
        t.view(torch.int16 if t.element_size() == 2 else torch.int32).fill_(-1)
    for p in list(per_rank) + [rest]:
        if len(p.segments):
            tm.execute(p, a, b, stream)
    torch.cuda.synchronize()
    bad, first = b.verify_synthetic(SEED, bf16=backup is None, vocab_rows=vocab_rows)
    if bad:
        print(f"[bench] shares verification FAILED: {bad} elements, first {first}", file=sys.stderr)
        return 3

    def timed(p):
        for _ in range(args.warmup):
            tm.execute(p, a, b, stream)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            tm.execute(p, a, b, stream)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps

    whole_ms = timed(plan)
    rows = []
    for g, p in enumerate(per_rank):
        if not len(p.segments):
            rows.append({"rank": g, "segments": 0})
            continue
        ms = timed(p)
        fp32, param = pull_bytes(p.segments, ls)
        local = int(fp32[g]) if g < len(fp32) else 0
        remote = int(fp32.sum()) - local + param
        rows.append({"rank": g, "segments": int(len(p.segments)), "payload_bytes": p.payload_bytes,
                     "read_bytes": p.read_bytes, "ms": round(ms, 4),
                     "traffic_gbps": round(p.traffic_bytes / (ms / 1e3) / 1e9, 1),
                     "frac_of_hbm_peak": round(p.traffic_bytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
                     "read_local_bytes": local, "read_remote_bytes": remote,
                     "remote_at_xgmi_ingress_ms": round(remote / (XGMI_INGRESS_GBPS * 1e9) * 1e3, 3)})
    timed_rows = [r for r in rows if r.get("ms")]
    out = {"what": "each destination rank's share of the copy plan timed alone on one GPU, every source in "
                   "its HBM; with one rank per GPU, share g is GPU g's part and its remote reads come over xGMI",
           "workload": desc, "kind": kind, "steps": args.steps, "warmup": args.warmup,
           "whole_plan_ms": round(whole_ms, 4),
           "whole_plan_gbps": round(plan.traffic_bytes / (whole_ms / 1e3) / 1e9, 1),
           "sum_of_shares_ms": round(sum(r["ms"] for r in timed_rows), 4),
           "max_share_ms": max((r["ms"] for r in timed_rows), default=0.0),
           "bf16_remainder_segments": int(len(rest.segments)),
           "verified_bit_exact": True, "launch": launch_shape(), "shares": rows}
    print(json.dumps(out), flush=True)
    return 0


def launch_shape():
    """The launch shape in effect (emrs_get_tuning), as the JSON line reports it."""
    from elasticmegatron_amd import _native

    t = _native.get_tuning()
    if t.persistent:
        return {"grid": "persistent", "blocks_per_cu": t.blocks_per_cu, "run": t.run, "xcd_remap": t.xcd_remap,
                "nontemporal": t.nontemporal}
    return {"grid": "one workgroup per piece", "lanes": t.lanes, "units_per_lane": t.units,
            "piece_bytes": 16 * t.lanes * t.units, "chunk_index": t.chunk_index, "warm_tables": t.warm_tables,
            "xcd_remap": t.xcd_remap,
            "buffer_ops": t.buffer_ops, "nontemporal": t.nontemporal}


def alternate_rounds(runs, stream, rounds=3, reps=5):
    """{name: [ms per launch of each round]}: each run's ``reps`` launches after one untimed one,
    the runs taking turns for ``rounds`` rounds, so that they compare on the same allocations in
    one process, without the spread of placements between processes."""
    import torch

    out = {name: [] for name in runs}
    for _ in range(rounds):
        for name, run in runs.items():
            run()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                run()
            e1.record(stream)
            torch.cuda.synchronize()
            out[name].append(round(e0.elapsed_time(e1) / reps, 4))
    return out


def read_ceiling(a, b, with_param, stream):
    """(ms, bytes) of emrs_xor_checksum over every arena the verification reads, in this process: the
    placement of the arenas moves a read-heavy launch by several percent between processes."""
    import torch

    from elasticmegatron_amd import _native

    word = torch.zeros(1, dtype=torch.int32, device=a.main.device)
    arenas = [a.main, a.exp_avg, a.exp_avg_sq, b.main, b.exp_avg, b.exp_avg_sq] + ([b.param] if with_param else [])
    spans = [(t.data_ptr(), t.numel() * t.element_size() // 16 * 16) for t in arenas]
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for p, n in spans:
        _native.xor_checksum(p, n, word.data_ptr(), stream.cuda_stream)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1), sum(n for _, n in spans)


def copy_ceiling(a, b, stream, traffic_gbps, read_bytes, write_bytes, reps=5):
    """What the very allocations the reshard ran on can do (physical placement moves every figure
    together), with the same 16-byte non-temporal accesses:

    - a plain contiguous copy of the source main arena into the destination one, by copy_plan_kernel;
    - write-only: the same kernel zero-filling the destination main arena (no reads), with one
      workgroup per 4 KB chunk whatever the launch shape (a workgroup that only stores 1 KB is so
      short that the rate of launching workgroups, not the memory, would bound the figure), in the
      faster of two shapes: 64 lanes of four units or 256 lanes of one;
    - read-only: emrs_xor_checksum over the source main arena (no writes);
    - both main arenas read together, as a comparison reads them: the plan check of that copy;
    - the workload's own read and write bytes moved one direction after the other at those two
      rates, a figure a kernel that overlaps reads with writes can beat.
    """
    import numpy as np
    import torch

    from elasticmegatron_amd import _native
    from elasticmegatron_amd.resharding.layout import SEG_ZERO_FILL, SEGMENT_DTYPE

    n = min(a.main.numel(), b.main.numel())

    def timed(run):
        for _ in range(2):
            run()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            run()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    t = np.zeros(1, dtype=SEGMENT_DTYPE)
    t[0] = (0, 0, 4, 0, 0, 0, n, 1, 0, 0, 0, 0, 0, 0)
    copy = _native.Plan(t, [n * 4], [n * 4])
    ms = timed(lambda: copy.execute([a.main.data_ptr()], [b.main.data_ptr()], stream.cuda_stream))
    t[0]["flags"] = SEG_ZERO_FILL
    fill = _native.Plan(t, [n * 4], [n * 4])
    tu = _native.get_tuning()
    shape = dict(blocks_per_cu=tu.blocks_per_cu, nontemporal=bool(tu.nontemporal), xcd_remap=tu.xcd_remap,
                 run=tu.run, persistent=bool(tu.persistent), lanes=tu.lanes, buffer_ops=bool(tu.buffer_ops),
                 chunk_index=bool(tu.chunk_index), warm_tables=bool(tu.warm_tables))
    w_shapes = {}
    try:
        for name, lanes, units in (("64x4", 64, 0), ("256x1", 256, 1)):   # one workgroup per chunk
            _native.set_tuning(**dict(shape, lanes=lanes), units=units)
            w_shapes[name] = timed(lambda: fill.execute([a.main.data_ptr()], [b.main.data_ptr()], stream.cuda_stream))
    finally:
        _native.set_tuning(**shape, units=tu.units)
    w_ms = min(w_shapes.values())
    word = torch.zeros(1, dtype=torch.int32, device=a.main.device)
    r_ms = timed(lambda: _native.xor_checksum(a.main.data_ptr(), n * 4, word.data_ptr(), stream.cuda_stream))
    # Reading both arenas together, as a comparison does: the plan's own check of the contiguous
    # copy just made (the destination now equals the source, so only its bit-level pass runs).
    both = [a.main.data_ptr()], [b.main.data_ptr()]
    copy.execute(*both, stream.cuda_stream)     # the write-only pass zeroed the destination
    if int(copy.compare(*both, stream=stream.cuda_stream)["mismatches"][0]):
        raise RuntimeError("the contiguous copy differs from its source")
    two = []
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        copy.compare(*both, stream=stream.cuda_stream)
        two.append((time.perf_counter() - t0) * 1e3)
    two_ms = sorted(two)[len(two) // 2]
    gbps = 2 * n * 4 / (ms / 1e3) / 1e9
    w_gbps, r_gbps = n * 4 / (w_ms / 1e3) / 1e9, n * 4 / (r_ms / 1e3) / 1e9
    serial = (read_bytes + write_bytes) / (read_bytes / r_gbps + write_bytes / w_gbps)
    return {"gbps": round(gbps, 1), "bytes_per_launch": 2 * n * 4, "ms": round(ms, 4),
            "what": "one contiguous copy of the main arena by copy_plan_kernel, same allocations",
            "reshard_frac_of_copy": round(traffic_gbps / gbps, 4),
            "read_only_gbps": round(r_gbps, 1), "write_only_gbps": round(w_gbps, 1),
            "write_only_gbps_by_shape": {k: round(n * 4 / (v / 1e3) / 1e9, 1) for k, v in w_shapes.items()},
            "two_arena_read_gbps": round(2 * n * 4 / (two_ms / 1e3) / 1e9, 1),
            "two_arena_read_what": "emrs_plan_compare of the contiguous copy (source and destination main arenas "
                                   "read together; wall time, median of the repetitions)",
            "serial_read_then_write_gbps": round(serial, 1),
            "reshard_frac_of_serial": round(traffic_gbps / serial, 4)}


def reshard_end_to_end(a, spec, src, dst, repad, tm, no_verify, reps=3):
    """ElasticMegatronManager.reshard wall time with the plan cached: allocation of the new
    state, the launch, release of the old optimizer state.  Two warm-up round trips first."""
    import logging

    import torch

    from elasticmegatron_amd import ElasticMegatronManager

    log = logging.getLogger("bench.reshard")
    log.propagate = False
    log.addHandler(logging.NullHandler())
    mgr = ElasticMegatronManager([src, dst], spec, training_state=a, repad_vocab=repad)
    mgr.transfer_manager = tm
    del a
    wall, execu = [], []
    for i in range(2 + reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        mgr.reshard(new_parallel_strategy=dst, logger=log)
        torch.cuda.synchronize()
        if i >= 2:
            wall.append((time.perf_counter() - t0) * 1e3)
            execu.append(mgr.last_transfer_ms)
        if i < 1 + reps:
            mgr.reshard(new_parallel_strategy=src, logger=log)
    st = mgr.training_state
    res = {"wall_ms": round(sorted(wall)[len(wall) // 2], 3), "executor_ms": round(sorted(execu)[len(execu) // 2], 3),
           "reps": reps}
    if not no_verify:
        vocab_rows = mgr.space_for(src).spec.padded_vocab_size if repad else None
        res["verified_bit_exact"] = st.verify_synthetic(SEED, vocab_rows=vocab_rows)[0] == 0
    # Hand back a state laid out as the source for anything after this.
    mgr.reshard(new_parallel_strategy=src, logger=log)
    return mgr.training_state, res


def copy_calibration(args, dev, stream):
    """One contiguous segment of known size: the reference point for HBM counters.

    The launch shape is the one the flags select, except that the workgroups find their segment by
    search rather than in the plan's chunk table, so that the kernel reads exactly the copied bytes.
    """
    import numpy as np
    import torch

    from elasticmegatron_amd import _native
    from elasticmegatron_amd.resharding.layout import SEGMENT_DTYPE

    _native.set_tuning(args.blocks_per_cu, bool(args.nontemporal), args.xcd_remap, args.run,
                       bool(args.persistent), args.lanes, args.units, chunk_index=False)
    n = int(args.copy_calibration_gib * (1 << 30)) // 16 * 4
    a = torch.ones(n, dtype=torch.float32, device=dev)
    b = torch.empty(n, dtype=torch.float32, device=dev)
    t = np.zeros(1, dtype=SEGMENT_DTYPE)
    t[0] = (0, 0, 4, 0, 0, 0, n, 1, 0, 0, 0, 0, 0, 0)
    plan = _native.Plan(t, [n * 4], [n * 4])
    if args.shape_sweep:
        return copy_shapes(args, plan, a, b, stream)
    for _ in range(args.warmup):
        plan.execute([a.data_ptr()], [b.data_ptr()], stream.cuda_stream)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.steps):
        plan.execute([a.data_ptr()], [b.data_ptr()], stream.cuda_stream)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    print(json.dumps({"copy_bytes": n * 4, "ms": round(ms, 4),
                      "traffic_GBps": round(2 * n * 4 / (ms / 1e3) / 1e9, 1)}), flush=True)
    return 0


def copy_shapes(args, plan, a, b, stream):
    """--copy-calibration-gib with --shape-sweep: the contiguous copy in each launch shape of the
    copy kernel, on the same two buffers, round after round; the fastest plain copy this kernel makes."""
    import torch

    from elasticmegatron_amd import _native

    rows = [{"shape": shp or "default", "ms": []} for shp in args.shape_sweep]
    try:
        for _ in range(args.rounds):
            for shp, row in zip(args.shape_sweep, rows):
                _native.set_tuning(**shp)
                b.zero_()
                for _ in range(args.warmup):
                    plan.execute([a.data_ptr()], [b.data_ptr()], stream.cuda_stream)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                e0.record(stream)
                for _ in range(args.steps):
                    plan.execute([a.data_ptr()], [b.data_ptr()], stream.cuda_stream)
                e1.record(stream)
                torch.cuda.synchronize()
                if not torch.equal(a, b):
                    print(f"[bench] copy shape {shp}: the copy differs from its source", file=sys.stderr)
                    return 3
                row["ms"].append(round(e0.elapsed_time(e1) / args.steps, 4))
                row["launch"] = launch_shape()
    finally:
        _native.set_tuning()
    nbytes = 2 * a.numel() * a.element_size()
    for row in rows:
        row["best_TBps"] = round(nbytes / (min(row["ms"]) / 1e3) / 1e12, 3)
    print(json.dumps({"what": "one contiguous copy in each launch shape of the copy kernel, same buffers, "
                               "rounds alternating", "copy_bytes": nbytes // 2, "rounds": args.rounds,
                      "shapes": rows}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
