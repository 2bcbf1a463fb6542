"""Full-size switches on one GPU.

Every destination element is checked on the device against the seeded
generator (its expected value is a closed form of (parameter, kind,
full-tensor index)), the plan's own verification compares the destination
with the source, and the switch back to the source layout must reproduce the
source exactly (round trip = identity).  The destination starts filled with a
canary pattern, and every element the layout does not store (padding) must
still hold it afterwards.

The CPU oracle cannot run a whole model at these sizes, but it runs the
parameters where placement is hardest: the word embedding and the output
layer (the largest tensors, whose DP shards cross bucket boundaries), the
final norm, and the last transformer layer.  For the transfer switches
Oracle-1 (the reference's three-pass executor, transfer.py:36-341, restated
on CPU tensors) runs them; for the Group-ZeRO switch Oracle-1's redundant
backup (transfer.py:343-388) does, after every source rank's shard has been
made distinct so that the instance -> rank mapping shows.  The GPU's pieces
of those parameters must equal the oracle bit for bit.  Peak memory is two
layouts' worth of state.
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
from tests.helpers import CANARY32, fill_canaries, padding_damage, perturb_per_rank

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


ORACLE_NAMES = ("embedding.word_embeddings.weight", "decoder.final_layernorm.weight", "output_layer.weight")


def _oracle_params(spec, budget=250_000_000):
    """Ids of the word embedding, final norm and output layer, and of the last transformer layer's
    parameters in order up to ``budget`` elements (Mixtral's experts exceed it)."""
    from oracle import model

    inv = model.inventory(spec)
    last = spec.num_layers - 1
    params, total = {p["id"] for p in inv if p["name"] in ORACLE_NAMES}, 0
    layer = False
    for p in inv:
        if p["layer"] == last and (not layer or total + model.numel(p["shape"]) <= budget):
            params.add(p["id"])
            total += model.numel(p["shape"])
            layer = True
    return inv, params


def _device_pieces(layout, state, params, bf16=True):
    got32, gotbf = {}, {}
    space = layout.space
    for pid in params:
        vp = space.all_virtual_params[pid]
        for h in layout.fp32_holders(vp):
            n = h.hi - h.lo
            got32[(h.rank, pid)] = {k: t[h.offset:h.offset + n].cpu().numpy()
                                    for k, t in zip(("main", "exp_avg", "exp_avg_sq"),
                                                    (state.main, state.exp_avg, state.exp_avg_sq))}
        if bf16:
            for h in layout.bf16_holders(vp):
                n = h.hi - h.lo
                gotbf[(layout.shard_keys[h.rank], pid)] = \
                    state.param[h.offset:h.offset + n].view(torch.int16).cpu().numpy().view(np.uint16)
    return got32, gotbf


def _check_against_oracle1(spec, src, dst, layout, state):
    """Oracle-1's transfer of the word embedding, final norm, output layer and last layer, against
    the same pieces of the device state, bit for bit."""
    from oracle import model
    from oracle import transfer as oracle1
    from oracle.plan import Strat
    from tests.helpers import compare

    inv, params = _oracle_params(spec)
    S, D = Strat.of(src), Strat.of(dst)
    world = oracle1.build_src_world(inv, spec, S, SEED, params)
    dw, dbf, _ = oracle1.transfer(inv, spec, S, D, world, params)
    want32 = oracle1.flatten(dw)
    del world, dw
    got32, gotbf = _device_pieces(layout, state, params)
    total = sum(model.numel(p["shape"]) for p in inv if p["id"] in params)
    print(f"oracle-1: {len(params)} params, {total} elements", flush=True)
    assert got32 and gotbf
    assert compare(got32, gotbf, want32, dbf) == []


def _check_backup_against_oracle1(spec, src, dst, a, b, tm, plan, scale_up):
    """Oracle-1's redundant backup from a source whose ranks hold distinct shards, against the
    device.  The source and destination are restored afterwards."""
    from oracle import model
    from oracle import transfer as oracle1
    from oracle.plan import Strat
    from tests.helpers import compare

    perturb_per_rank(a)
    tm.execute(plan, a, b)
    inv, params = _oracle_params(spec)
    S, D = Strat.of(src), Strat.of(dst)
    world = oracle1.build_src_world(inv, spec, S, SEED, params)
    perturb_per_rank(world)
    want = oracle1.flatten(oracle1.redundant_backup(inv, spec, S, D, world, scale_up, params))
    del world
    got, _ = _device_pieces(b.layout, b, params, bf16=False)
    total = sum(model.numel(p["shape"]) for p in inv if p["id"] in params)
    print(f"oracle-1 redundant backup: {len(params)} params, {total} elements", flush=True)
    assert got
    assert compare(got, {}, want, {}) == []
    perturb_per_rank(a)  # XOR again: the seeded values are back
    tm.execute(plan, a, b)


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
        if backup is None:
            fill_canaries(b)
        else:  # the bf16 arena is shared with the source: only the fp32 arenas start as canaries
            for t in (b.main, b.exp_avg, b.exp_avg_sq):
                t.view(torch.int32).fill_(CANARY32)
        tm.execute(fwd, a, b)
        bad, first = b.verify_synthetic(SEED, vocab_rows=vocab_rows)
        assert bad == 0, first
        assert padding_damage(b, bf16=backup is None) == 0, "padding was written"
        report = tm.verify(a, b, kind)  # the plan's own check, against the source state
        assert report.bit_exact, report.lines()[:5]
        if kind == "transfer" and not repad:  # the reference keeps the padded vocabulary fixed
            _check_against_oracle1(spec, src, dst, ld, b)
        elif backup is not None:
            _check_backup_against_oracle1(spec, src, dst, a, b, tm, fwd, backup)
            assert b.verify_synthetic(SEED)[0] == 0
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
