"""An exporting process for a synthetic training state.

    python -m elasticmegatron_amd.transfer.ipc_export --model-spec JSON --strategy JSON [--seed N]
        [--granule-bytes B] [--device D] [--misc JSON] [--start-from JSON]

Stands in for the old training process of a hand-off (the reference's
send_training_state, elastic_megatron/transfer/ipc_manager.py:54-132): it
allocates a :class:`~.ipc_manager.SharedTrainingState`, fills it with the
seeded synthetic values, writes the payload as one line on stdout, and keeps
the memory until a release notice arrives on stdin (or stdin closes).  An
arena's own release notice (a staged switch releases the source arena by
arena) frees that arena's granules and is answered on stdout once the memory
is back with the driver.  With ``--start-from`` the state is filled in that
strategy first and reaches ``--strategy`` by one verified reshard in this
process, as a job that resharded before handing off.
"""

import json
import logging
import sys
from typing import Sequence

import torch

from ..megatron_manager.parallel_strategy import ParallelStrategy
from ..resharding.granules import DEFAULT_GRANULE_BYTES
from ..resharding.layout import ARENA_NAMES
from ..resharding.model_spec import ModelSpec
from ..resharding.virtual_param import build_virtual_model
from .ipc_manager import SharedTrainingState, notify_freed, send_training_state, wait_for_release


def main(argv: Sequence[str]) -> int:
    """An exporting process for a synthetic state: allocate, fill, send on stdout, wait for the
    release notice on stdin.  Stands in for the old training process of a hand-off."""
    import argparse

    ap = argparse.ArgumentParser(prog="python -m elasticmegatron_amd.transfer.ipc_export")
    ap.add_argument("--model-spec", required=True, help="ModelSpec fields as JSON")
    ap.add_argument("--strategy", required=True, help="ParallelStrategy fields as JSON")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--granule-bytes", type=int, default=DEFAULT_GRANULE_BYTES)
    ap.add_argument("--device", type=int, default=0)
    ap.add_argument("--misc", default="{}", help="JSON passed through in the payload")
    ap.add_argument("--start-from", default=None,
                    help="ParallelStrategy fields as JSON: fill the state in this strategy, then reach --strategy "
                         "by one verified reshard in this process")
    args = ap.parse_args(argv)

    spec = ModelSpec(**json.loads(args.model_spec))
    target = ParallelStrategy(**json.loads(args.strategy))
    dev = torch.device("cuda", args.device)
    torch.cuda.set_device(args.device)
    if args.start_from is None:
        state = SharedTrainingState.allocate(build_virtual_model(spec).layout(target), dev, args.granule_bytes)
        state.fill_synthetic(args.seed)
    else:
        from ..elastic_manager import ElasticMegatronManager

        mgr = ElasticMegatronManager([ParallelStrategy(**json.loads(args.start_from)), target], spec, device=dev,
                                     share_granule_bytes=args.granule_bytes)
        mgr.training_state.fill_synthetic(args.seed)
        # The perf line goes to the log, not to stdout, which carries the payload.
        state = mgr.reshard(target, logger=logging.getLogger("ipc_export"), verify=True)
    layout = state.layout
    print(f"[exporter] {len(state.buffers)} granules of {layout.strategy} filled", file=sys.stderr, flush=True)
    send_training_state(state, sys.stdout, misc=json.loads(args.misc))

    def free_arena(name: str) -> None:
        state.release_kind(ARENA_NAMES.index(name))
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        print(f"[exporter] {name} freed", file=sys.stderr, flush=True)
        notify_freed(sys.stdout, name)

    released = wait_for_release(sys.stdin, on_arena=free_arena)
    print(f"[exporter] {'released' if released else 'channel closed'}; exiting", file=sys.stderr, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
