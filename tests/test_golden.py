"""Golden fixtures of the tiny LLaMA-2 switches (tests/golden/tiny_llama2.json).

Pins the oracle (generator, plan and executor restatements) against its own
recorded outputs, and the product's plan against the same digests.
"""

import json
import os

import numpy as np
import pytest

from elasticmegatron_amd.resharding.lowering import lower_transfer
from elasticmegatron_amd.resharding.model_spec import tiny_llama2
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from tests.golden import make_golden
from tests.helpers import execute_numpy, extract, new_arenas, piece_fill_numpy

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def golden():
    with open(os.path.join(HERE, "golden", "tiny_llama2.json")) as f:
        return json.load(f)


def test_oracle_reproduces_golden(golden):
    assert make_golden.run() == golden


def test_product_plan_reproduces_golden(golden):
    space = build_virtual_model(tiny_llama2())
    for sw, a, b in zip(golden["switches"], make_golden.SEQ, make_golden.SEQ[1:]):
        ls, ld = space.layout(a), space.layout(b)
        src, dst = new_arenas(ls), new_arenas(ld)
        piece_fill_numpy(ls.pieces(), src, golden["seed"])
        s32, _ = extract(ls, src)
        assert {f"{g}/{pid}/{k}": make_golden.digest(v.view(np.float32)) for (g, pid), kinds in s32.items()
                for k, v in kinds.items()} == sw["src_pieces"]
        execute_numpy(lower_transfer(ls, ld), src, dst)
        d32, dbf = extract(ld, dst)
        assert {f"{g}/{pid}/{k}": make_golden.digest(v.view(np.float32)) for (g, pid), kinds in d32.items()
                for k, v in kinds.items()} == sw["dst_fp32"]
        assert {f"{'-'.join(map(str, key))}/{pid}": make_golden.digest(v) for (key, pid), v in dbf.items()} \
            == sw["dst_bf16"]
