"""Full-size switches on one GPU.

Every destination element is checked on the device against the seeded
generator (its expected value is a closed form of (parameter, kind,
full-tensor index)), the plan's own verification compares the destination
with the source, and the switch back to the source layout must reproduce the
source exactly (round trip = identity).  The CPU oracle cannot run a whole
model at these sizes, but it runs one layer: for the transfer switches,
Oracle-1 (the reference's three-pass executor, transfer.py:36-341, restated
on CPU tensors) runs the parameters of the last transformer layer, about
250M elements, and the GPU result must equal it bit for bit.  Peak memory is
two layouts' worth of state.
"""

import gc

import numpy as np
import pytest
import torch

from elasticmegatron_amd import ParallelStrategy as PS
from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding import model_spec as ms
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager

pytestmark = pytest.mark.gpu
SEED = 1234

CASES = [
    pytest.param(ms.llama2_7b, PS(8, 1, 1), PS(8, 4, 1), id="llama2-7b-tp1dp8-tp4dp2"),
    pytest.param(ms.llama3_8b, PS(8, 2, 2), PS(8, 4, 1), id="llama3-8b-tp2pp2dp2-tp4pp1dp2"),
    pytest.param(ms.llama3_8b, PS(8, 2, 2), PS(8, 4, 1), True, id="llama3-8b-tp2pp2dp2-tp4pp1dp2-repad"),
    pytest.param(ms.mixtral_8x7b_slice, PS(8, 1, 1, expert_model_parallel_size=4),
                 PS(8, 1, 1, expert_model_parallel_size=8), id="mixtral-4l-ep4-ep8"),
    pytest.param(ms.llama2_7b, PS(8, 1, 1), PS(6, 1, 1), id="llama2-7b-dp8-dp6"),
    pytest.param(ms.llama2_7b, PS(6, 1, 1), PS(12, 1, 1, num_distributed_optimizer_instances=2),
                 id="llama2-7b-groupzero-1-2"),
]


def _release():
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _check_layer_against_oracle1(spec, src, dst, layout, state, budget=250_000_000):
    """Oracle-1 on the last transformer layer's parameters (in order, up to ``budget`` elements), and
    the same pieces of the device state copied back, compared bit for bit."""
    from oracle import model
    from oracle import transfer as oracle1
    from oracle.plan import Strat
    from tests.helpers import compare

    inv = model.inventory(spec)
    last = spec.num_layers - 1
    params, total = set(), 0
    for p in inv:
        if p["layer"] == last and (not params or total + model.numel(p["shape"]) <= budget):
            params.add(p["id"])
            total += model.numel(p["shape"])
    S, D = Strat.of(src), Strat.of(dst)
    world = oracle1.build_src_world(inv, spec, S, SEED, params)
    dw, dbf, _ = oracle1.transfer(inv, spec, S, D, world, params)
    want32 = oracle1.flatten(dw)
    got32, gotbf = {}, {}
    space = layout.space
    for pid in params:
        vp = space.all_virtual_params[pid]
        for h in layout.fp32_holders(vp):
            n = h.hi - h.lo
            got32[(h.rank, pid)] = {k: t[h.offset:h.offset + n].cpu().numpy()
                                    for k, t in zip(("main", "exp_avg", "exp_avg_sq"),
                                                    (state.main, state.exp_avg, state.exp_avg_sq))}
        for h in layout.bf16_holders(vp):
            n = h.hi - h.lo
            gotbf[(layout.shard_keys[h.rank], pid)] = \
                state.param[h.offset:h.offset + n].view(torch.int16).cpu().numpy().view(np.uint16)
    print(f"oracle-1 on layer {last}: {len(params)} params, {total} elements", flush=True)
    assert got32 and gotbf
    assert compare(got32, gotbf, want32, dbf) == []


@pytest.mark.parametrize("factory,src,dst,repad", [p if len(p.values) == 4 else
                                                   pytest.param(*p.values, False, id=p.id) for p in CASES])
def test_full_size_switch_and_round_trip(gpu_device, factory, src, dst, repad):
    spec = factory()
    print(f"case {spec.name}: {src} -> {dst} repad {repad}", flush=True)
    backup = PS.is_redundant_backup(src, dst)
    kind = "transfer" if backup is None else ("backup_up" if backup else "backup_down")
    back_kind = "transfer" if backup is None else ("backup_down" if backup else "backup_up")
    if repad:  # Megatron's padded vocabulary at each TP size; new padding rows are zero
        ls, ld = (build_virtual_model(spec.with_padded_vocab(spec.padded_vocab_for_tp(
            s.tensor_model_parallel_size))).layout(s) for s in (src, dst))
        assert ld.space.spec.padded_vocab_size > ls.space.spec.padded_vocab_size
    else:
        space = build_virtual_model(spec)
        ls, ld = space.layout(src), space.layout(dst)
    vocab_rows = ls.space.spec.padded_vocab_size if repad else None
    tm = TransferManager()
    fwd = tm.compile(ls, ld, kind)
    rev = tm.compile(ld, ls, back_kind)
    assert fwd.native.stats().scalar_bytes == 0, "every segment should take the 16-byte path"
    try:
        a = TrainingState.allocate(ls, gpu_device)
        b = TrainingState.allocate(ld, gpu_device, param=a.param if backup is not None else None)
        a.fill_synthetic(SEED)
        tm.execute(fwd, a, b)
        bad, first = b.verify_synthetic(SEED, vocab_rows=vocab_rows)
        assert bad == 0, first
        report = tm.verify(a, b, kind)  # the plan's own check, against the source state
        assert report.bit_exact, report.lines()[:5]
        if kind == "transfer" and not repad:  # the reference keeps the padded vocabulary fixed
            _check_layer_against_oracle1(spec, src, dst, ld, b)
        # Round trip into fresh storage: must reproduce every source element.
        param = a.param
        del a
        _release()
        a2 = TrainingState.allocate(ls, gpu_device, param=param if backup is not None else None)
        if backup is None:
            a2.param.zero_()
        for t in (a2.main, a2.exp_avg, a2.exp_avg_sq):
            t.fill_(float("nan"))
        tm.execute(rev, b, a2)
        bad, first = a2.verify_synthetic(SEED)
        assert bad == 0, first
    finally:
        a = b = a2 = param = None  # noqa: F841
        _release()
