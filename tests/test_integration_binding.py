"""The ctypes binding that INTEGRATION.md gives a maintainer, run as written.

The Python block under "The Python-side binding a maintainer would add" is
executed with its library name pointed at the in-tree build.  On the CPU its
segment record and flag values must equal the header's (as the product's
binding states them), and it must create plans and surface the library's
errors.  On the GPU the tiny LLaMA-2 switches run through it (the first one
prepared ahead, as the meta-device pass would) must reproduce the golden
digests (tests/golden/tiny_llama2.json), which the oracle is pinned against.
"""

import json
import os
import re

import numpy as np
import pytest

from elasticmegatron_amd import _native
from elasticmegatron_amd.resharding import layout as lay
from elasticmegatron_amd.resharding.lowering import lower_transfer
from elasticmegatron_amd.resharding.model_spec import tiny_llama2
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from tests.golden import make_golden
from tests.helpers import extract, new_arenas, piece_fill_numpy

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_NAME = 'ctypes.CDLL("libemrs.so")'


def _binding():
    with open(os.path.join(ROOT, "INTEGRATION.md")) as f:
        text = f.read()
    section = text.split("## The Python-side binding a maintainer would add", 1)[1]
    code = re.search(r"```python\n(.*?)```", section, re.S).group(1)
    assert code.count(LIB_NAME) == 1
    code = code.replace(LIB_NAME, f"ctypes.CDLL({_native.LIB_PATH!r})")
    ns = {}
    exec(compile(code, "INTEGRATION.md (binding)", "exec"), ns)
    return ns


@pytest.fixture(scope="module")
def binding():
    _native.load()  # fails loudly when the library is not built
    return _binding()


def _sizes(layout):
    return [layout.fp32_numel * 4] * 3 + [layout.bf16_numel * 2]


def test_binding_record_and_flags_match_the_header(binding):
    seg = binding["SEGMENT"]
    assert seg.itemsize == 88 == lay.SEGMENT_DTYPE.itemsize
    assert seg.names == lay.SEGMENT_DTYPE.names
    assert [seg.fields[n][1] for n in seg.names] == [lay.SEGMENT_DTYPE.fields[n][1] for n in seg.names]
    assert [seg.fields[n][0] for n in seg.names] == [lay.SEGMENT_DTYPE.fields[n][0] for n in seg.names]
    assert (binding["SEG_CAST_BF16"], binding["SEG_ZERO_FILL"], binding["SEG_DUP"]) == \
        (lay.SEG_CAST_BF16, lay.SEG_ZERO_FILL, lay.SEG_DUP)


def test_binding_creates_plans_and_reports_errors(binding):
    space = build_virtual_model(tiny_llama2())
    a, b = make_golden.SEQ[0], make_golden.SEQ[1]
    ls, ld = space.layout(a), space.layout(b)
    table = lower_transfer(ls, ld)
    h = binding["plan_create"](table, _sizes(ls), _sizes(ld))
    assert h.value
    binding["lib"].emrs_plan_destroy(h)
    bad = table.copy()
    bad[0]["src_off"] = ls.fp32_numel  # runs past the end of its source buffer
    with pytest.raises(RuntimeError, match="source range exceeds its buffer"):
        binding["plan_create"](bad, _sizes(ls), _sizes(ld))


@pytest.mark.gpu
def test_binding_runs_the_golden_switches(gpu_device, binding):
    import torch

    with open(os.path.join(ROOT, "tests", "golden", "tiny_llama2.json")) as f:
        golden = json.load(f)
    space = build_virtual_model(tiny_llama2())
    lib = binding["lib"]
    for i, (sw, a, b) in enumerate(zip(golden["switches"], make_golden.SEQ, make_golden.SEQ[1:])):
        print(f"binding switch {i}: TP{a.tensor_model_parallel_size} -> TP{b.tensor_model_parallel_size}",
              flush=True)
        ls, ld = space.layout(a), space.layout(b)
        src, dst = new_arenas(ls), new_arenas(ld)
        piece_fill_numpy(ls.pieces(), src, golden["seed"])
        to_dev = [torch.from_numpy(x.view(np.int32) if x.dtype == np.uint32 else x.view(np.int16)).to(gpu_device)
                  for x in src]
        out = [torch.from_numpy(x.view(np.int32) if x.dtype == np.uint32 else x.view(np.int16)).to(gpu_device)
               for x in dst]
        h = binding["plan_create"](lower_transfer(ls, ld), _sizes(ls), _sizes(ld))
        try:
            if i == 0:
                binding["plan_prepare"](h, torch.cuda.current_stream(gpu_device))
            binding["plan_execute"](h, to_dev, out, torch.cuda.current_stream(gpu_device))
            torch.cuda.synchronize(gpu_device)
        finally:
            lib.emrs_plan_destroy(h)
        got = [t.cpu().numpy().view(np.uint32 if t.dtype == torch.int32 else np.uint16) for t in out]
        d32, dbf = extract(ld, got)
        assert {f"{g}/{pid}/{k}": make_golden.digest(v.view(np.float32)) for (g, pid), kinds in d32.items()
                for k, v in kinds.items()} == sw["dst_fp32"]
        assert {f"{'-'.join(map(str, key))}/{pid}": make_golden.digest(v) for (key, pid), v in dbf.items()} \
            == sw["dst_bf16"]
