"""Writes tests/golden/tiny_llama2.json: digests of Oracle-1's outputs on the
tiny LLaMA-2 switches TP2DP4 -> TP1DP8 -> TP4DP2 (world 8, seed 1234).

The reference ships no golden vectors for this path and cannot run here
(it needs Megatron-core and a multi-GPU world), so these fixtures are the
oracle's own outputs: they pin regressions of the generator, the plan
restatement and the executor restatement.

    python tests/golden/make_golden.py
"""

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy as PS  # noqa: E402
from elasticmegatron_amd.resharding.model_spec import tiny_llama2  # noqa: E402
from oracle import model  # noqa: E402
from oracle import transfer as oracle1  # noqa: E402
from oracle.plan import Strat  # noqa: E402

SEED = 1234
SEQ = [PS(8, 2, 1), PS(8, 1, 1), PS(8, 4, 1)]


def digest(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:24]


def run():
    spec = tiny_llama2()
    inv = model.inventory(spec)
    out = {"seed": SEED, "model": spec.name, "switches": []}
    for a, b in zip(SEQ, SEQ[1:]):
        S, D = Strat.of(a), Strat.of(b)
        world = oracle1.build_src_world(inv, spec, S, SEED)
        src = {f"{g}/{pid}/{k}": digest(info.tensors[i].numpy())
               for pid, infos in world.items() for g, info in infos.items()
               for i, k in enumerate(oracle1.KINDS)}
        dw, dbf, mb = oracle1.transfer(inv, spec, S, D, world)
        fp32 = {f"{g}/{pid}/{k}": digest(v) for (g, pid), kinds in oracle1.flatten(dw).items()
                for k, v in kinds.items()}
        bf16 = {f"{'-'.join(map(str, key))}/{pid}": digest(v) for (key, pid), v in dbf.items()}
        flat = oracle1.flatten(dw)
        first = min(flat)
        sample = {k: flat[first][k][:4].view(np.uint32).tolist() for k in oracle1.KINDS}
        out["switches"].append({
            "src": [a.world_size, a.tensor_model_parallel_size, a.pipeline_model_parallel_size],
            "dst": [b.world_size, b.tensor_model_parallel_size, b.pipeline_model_parallel_size],
            "src_pieces": src, "dst_fp32": fp32, "dst_bf16": bf16,
            "first_piece": list(first), "first_piece_first4_bits": sample,
            "max_cross_rank_bytes": max(mb.cross_rank_bytes.values()),
        })
    return out


if __name__ == "__main__":
    with open(os.path.join(HERE, "tiny_llama2.json"), "w") as f:
        json.dump(run(), f, indent=0, sort_keys=True)
    print("wrote", os.path.join(HERE, "tiny_llama2.json"))
