"""GPU parity of the native copy-plan executor (bit-exact).

Small models: the kernel's output against Oracle-1 (the reference's
three-pass executor restated on CPU torch tensors).  Hand-made segment
tables: against the numpy reference semantics of emrs_plan_execute, covering
the vector, scalar, strided and split-alignment paths.
"""

import numpy as np
import pytest
import torch

from elasticmegatron_amd import _native
from elasticmegatron_amd.megatron_manager.training_state import TrainingState
from elasticmegatron_amd.resharding.layout import SEGMENT_DTYPE
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.transfer import TransferManager
from oracle import model
from oracle import transfer as oracle1
from tests.helpers import (REPAD_CASES, SEED, SMALL_CASES, bf16_rne_bits, compare, extract, fill_canaries,
                           new_arenas, padding_damage, piece_fill_numpy, repad_spaces, strat)

pytestmark = pytest.mark.gpu


def _host_arenas(state):
    torch.cuda.synchronize()
    out = [t.cpu().view(torch.int32).numpy().view(np.uint32) for t in state.arenas()[:3]]
    out.append(state.param.cpu().view(torch.int16).numpy().view(np.uint16))
    return out


def test_device_generator_matches_numpy(gpu_device):
    """emrs_synth_fill == the numpy generator, every stored element of a tiny layout."""
    from elasticmegatron_amd.resharding.model_spec import tiny_llama2
    from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy as PS

    space = build_virtual_model(tiny_llama2())
    lay = space.layout(PS(8, 2, 1))
    st = TrainingState.allocate(lay, gpu_device)
    for t in st.arenas():
        t.zero_()
    st.fill_synthetic(SEED)
    got = _host_arenas(st)
    want = new_arenas(lay, fill=0)
    piece_fill_numpy(lay.pieces(), want, SEED)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)
    bad, first = st.verify_synthetic(SEED)
    assert bad == 0, first


def _switches():
    for name, factory, seq in SMALL_CASES:
        for a, b in zip(seq, seq[1:]):
            yield pytest.param(factory, a, b, id=f"{name}-{a.tensor_model_parallel_size}x"
                               f"{a.pipeline_model_parallel_size}x{a.world_size}-{b.tensor_model_parallel_size}x"
                               f"{b.pipeline_model_parallel_size}x{b.world_size}")


@pytest.mark.parametrize("factory,src,dst,bf16_source",
                         [p.values + ("cast",) for p in _switches()] +
                         [p.values + ("copy",) for p in list(_switches())[:4]])
def test_kernel_matches_oracle1(gpu_device, factory, src, dst, bf16_source):
    spec = factory()
    print(f"case {spec.name} {src} -> {dst} bf16 {bf16_source}", flush=True)
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    a = TrainingState.allocate(ls, gpu_device)
    b = TrainingState.allocate(ld, gpu_device)
    a.fill_synthetic(SEED)
    fill_canaries(b)  # every stored element must be overwritten, every padding element kept
    tm = TransferManager(check_disjoint=True, bf16_source=bf16_source)
    tm.transfer_optimizer_tensors(space, src=a, dst=b)
    got32, gotbf = extract(ld, _host_arenas(b))
    assert padding_damage(b) == 0

    inv = model.inventory(spec)
    S, D = strat(src), strat(dst)
    world = oracle1.build_src_world(inv, spec, S, SEED)
    dw, dbf, _ = oracle1.transfer(inv, spec, S, D, world)
    assert compare(got32, gotbf, oracle1.flatten(dw), dbf) == []
    bad, first = b.verify_synthetic(SEED)
    assert bad == 0, first


@pytest.mark.parametrize("factory,vocab,src,dst", REPAD_CASES)
@pytest.mark.parametrize("bf16_source", ["cast", "copy"])
def test_repad_kernel_matches_invariant(gpu_device, factory, vocab, src, dst, bf16_source):
    """Vocabulary re-padding: kept rows carry their values, new padding rows are zero."""
    from dataclasses import replace
    from oracle import canonical

    spec = replace(factory(), vocab_size=vocab)
    sa, sb = repad_spaces(spec, (src.tensor_model_parallel_size, dst.tensor_model_parallel_size))
    print(f"case {spec.name} vocab {sa.spec.padded_vocab_size} -> {sb.spec.padded_vocab_size} "
          f"{src} -> {dst} bf16 {bf16_source}", flush=True)
    ls, ld = sa.layout(src), sb.layout(dst)
    a = TrainingState.allocate(ls, gpu_device)
    b = TrainingState.allocate(ld, gpu_device)
    a.fill_synthetic(SEED)
    for t in b.arenas():
        t.fill_(0) if t.dtype != torch.float32 else t.fill_(float("nan"))
    TransferManager(check_disjoint=True, bf16_source=bf16_source).transfer_optimizer_tensors(None, src=a, dst=b)
    got32, gotbf = extract(ld, _host_arenas(b))
    want32, wantbf = canonical.world(model.inventory(sb.spec), sb.spec, strat(dst), SEED,
                                     vocab_rows=sa.spec.padded_vocab_size)
    assert compare(got32, gotbf, want32, wantbf) == []
    bad, first = b.verify_synthetic(SEED, vocab_rows=sa.spec.padded_vocab_size)
    assert bad == 0, first


def test_manager_repad_round_trip(gpu_device):
    """ElasticMegatronManager(repad_vocab=True): TP2PP2 -> TP4PP1 -> TP2PP2 is the identity."""
    from dataclasses import replace
    from elasticmegatron_amd import ElasticMegatronManager
    from tests.helpers import small_llama3

    spec = replace(small_llama3(), vocab_size=2300)
    seq = [dict(world_size=8, tensor_model_parallel_size=2, pipeline_model_parallel_size=2),
           dict(world_size=8, tensor_model_parallel_size=4, pipeline_model_parallel_size=1)]
    mgr = ElasticMegatronManager(seq, spec, device=gpu_device, repad_vocab=True)
    mgr.training_state.fill_synthetic(SEED)
    st = mgr.reshard(new_parallel_strategy=seq[1])
    assert st.layout.space.spec.padded_vocab_size == 2560
    assert st.verify_synthetic(SEED, vocab_rows=2304)[0] == 0
    st = mgr.reshard(new_parallel_strategy=seq[0])
    assert st.layout.space.spec.padded_vocab_size == 2304
    assert st.verify_synthetic(SEED)[0] == 0


@pytest.mark.parametrize("tuning", [dict(chunk_index=False), dict(units=4, chunk_index=False), dict(units=0),
                                    dict(units=2, chunk_index=False), dict(lanes=256, units=1, chunk_index=False),
                                    dict(buffer_ops=True, chunk_index=False), dict(xcd_remap=2, chunk_index=False),
                                    dict(units=4), dict(units=4, xcd_remap=2),
                                    dict(nontemporal=False), dict(lanes=128), dict(lanes=256),
                                    dict(lanes=256, nontemporal=False), dict(units=1), dict(units=2),
                                    dict(lanes=128, units=1), dict(units=1, nontemporal=False),
                                    dict(buffer_ops=True), dict(buffer_ops=True, nontemporal=False),
                                    dict(buffer_ops=True, units=1), dict(buffer_ops=True, lanes=256),
                                    dict(buffer_ops=True, lanes=128, units=2),
                                    dict(xcd_remap=False), dict(xcd_remap=2), dict(units=1, xcd_remap=2),
                                    dict(lanes=256, units=1, xcd_remap=2), dict(lanes=128, units=2, xcd_remap=2),
                                    dict(buffer_ops=True, xcd_remap=2), dict(nontemporal=False, xcd_remap=2),
                                    dict(persistent=True),
                                    dict(persistent=True, run=0), dict(persistent=True, run=0, xcd_remap=False),
                                    dict(persistent=True, run=1), dict(persistent=True, run=64),
                                    dict(persistent=True, blocks_per_cu=1),
                                    dict(persistent=True, nontemporal=False),
                                    dict(persistent=True, blocks_per_cu=3, run=7),
                                    dict(persistent=True, run=4, xcd_remap=False),
                                    dict(persistent=True, run=1, blocks_per_cu=1, xcd_remap=False)])
def test_launch_shape_does_not_change_results(gpu_device, tuning):
    """Every launch shape of emrs_set_tuning writes the same bits."""
    from elasticmegatron_amd.resharding.model_spec import tiny_llama2
    from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy as PS

    print(f"case tuning {tuning}", flush=True)
    space = build_virtual_model(tiny_llama2())
    ls, ld = space.layout(PS(8, 2, 1)), space.layout(PS(8, 4, 1))
    a = TrainingState.allocate(ls, gpu_device)
    a.fill_synthetic(SEED)
    outs = []
    try:
        for t in (dict(), tuning):
            _native.set_tuning(**t)
            b = TrainingState.allocate(ld, gpu_device)
            for x in b.arenas():
                x.fill_(0) if x.dtype != torch.float32 else x.fill_(float("nan"))
            TransferManager(check_disjoint=True).transfer_optimizer_tensors(None, src=a, dst=b)
            outs.append(_host_arenas(b))
    finally:
        _native.set_tuning()
    for x, y in zip(*outs):
        assert np.array_equal(x, y)
    assert _native.get_tuning().run == 4 and _native.get_tuning().persistent == 0


def _random_table(rng, n_segs, sizes):
    rows = []
    for _ in range(n_segs):
        eb = int(rng.choice([1, 2, 4, 8]))
        nb = [sz // eb for sz in sizes]
        r = int(rng.choice([1, 1, 2, 7, 33]))
        ln = int(rng.integers(1, 300))
        ss = ln + int(rng.integers(0, 40)) if r > 1 else 0
        ds = ln + int(rng.integers(0, 40)) if r > 1 else 0
        if rng.random() < 0.3 and r > 1:  # 16-byte friendly strided rows
            ln = (ln // (16 // eb) + 1) * (16 // eb)
            ss = ds = ln * 2
        src_ext = (r - 1) * ss + ln
        dst_ext = (r - 1) * ds + ln
        so = int(rng.integers(0, nb[0] - src_ext))
        do = int(rng.integers(0, nb[1] - dst_ext))
        if rng.random() < 0.5:  # co-aligned offsets exercise the head/body/tail split
            do = do - (do * eb) % 16 // eb + (so * eb) % 16 // eb
            do = max(0, min(do, nb[1] - dst_ext))
        cast = eb == 4 and rng.random() < 0.5
        dup = not cast and rng.random() < 0.4
        zero = 2 if rng.random() < 0.2 else 0  # zero fill: the source offset is ignored
        if zero and rng.random() < 0.5:
            so = int(rng.integers(0, 1 << 40))
        if cast:  # bf16 image into the second destination buffer
            aux_s = ln + int(rng.integers(0, 9)) if r > 1 else 0
            ao = int(rng.integers(0, sizes[1] // 2 - ((r - 1) * aux_s + ln)))
            rows.append((0, 0, eb, 1 | zero, so, do, ln, r, ss, ds, 1, 0, ao, aux_s))
        elif dup:  # unchanged copy into the second destination buffer
            aux_s = (ds if rng.random() < 0.5 else ln + int(rng.integers(0, 9))) if r > 1 else 0
            ext = (r - 1) * aux_s + ln
            ao = int(rng.integers(0, sizes[1] // eb - ext))
            if rng.random() < 0.6:  # co-aligned with the destination: vector and head/body/tail paths
                ao = ao - (ao * eb) % 16 // eb + (do * eb) % 16 // eb
                ao = max(0, min(ao, sizes[1] // eb - ext))
            rows.append((0, 0, eb, 4 | zero, so, do, ln, r, ss, ds, 1, 0, ao, aux_s))
        else:
            rows.append((0, 0, eb, zero, so, do, ln, r, ss, ds, 0, 0, 0, 0))
    t = np.zeros(len(rows), dtype=SEGMENT_DTYPE)
    t[:] = rows
    return t


@pytest.mark.parametrize("seed,tuning", [(0, {}), (1, {}), (2, {}), (3, dict(lanes=128)), (4, dict(lanes=256)),
                                         (5, dict(persistent=True)), (6, dict(lanes=256, nontemporal=False)),
                                         (7, dict(units=1)), (8, dict(units=2)), (9, dict(lanes=128, units=1)),
                                         (10, dict(buffer_ops=True)), (11, dict(buffer_ops=True, nontemporal=False)),
                                         (12, dict(buffer_ops=True, units=1)), (13, dict(chunk_index=False)),
                                         (14, dict(units=4, chunk_index=False)), (15, dict(units=0)),
                                         (13, dict(buffer_ops=True, lanes=256))])
def test_random_segments_match_numpy(gpu_device, seed, tuning):
    """Arbitrary element sizes, offsets and strides (scalar, split and vector paths), zero fills,
    bf16 images and duplicates, under each launch shape.

    Segments are applied in order and may overlap in the destination here, so
    each segment runs as its own plan and the numpy model applies the same
    sequence.
    """
    print(f"case random segments seed {seed} tuning {tuning}", flush=True)
    try:
        _native.set_tuning(**tuning)
        _random_segments_match_numpy(gpu_device, seed)
    finally:
        _native.set_tuning()


def _random_segments_match_numpy(gpu_device, seed):
    rng = np.random.default_rng(seed)
    nbytes = 1 << 20
    src_h = rng.integers(0, 256, nbytes, dtype=np.uint8)
    src = torch.from_numpy(src_h).to(gpu_device)
    fill = rng.integers(0, 256, nbytes, dtype=np.uint8)  # so that written zeros show
    dst = torch.from_numpy(fill).to(gpu_device)
    aux = torch.from_numpy(fill).to(gpu_device)
    want = fill.copy()
    want_aux = fill.copy()
    table = _random_table(rng, 40, (nbytes, nbytes))
    for s in table:
        one = np.array([s], dtype=SEGMENT_DTYPE)
        plan = _native.Plan(one, [nbytes], [nbytes, nbytes])
        plan.execute([src.data_ptr()], [dst.data_ptr(), aux.data_ptr()], torch.cuda.current_stream().cuda_stream)
        eb = int(s["elem_bytes"])
        a, b = src_h.view({1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[eb]), \
            want.view({1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[eb])
        for r in range(int(s["rows"])):
            so = int(s["src_off"]) + r * int(s["src_stride"])
            do = int(s["dst_off"]) + r * int(s["dst_stride"])
            vals = np.zeros(int(s["len"]), dtype=b.dtype) if int(s["flags"]) & 2 else a[so:so + int(s["len"])]
            b[do:do + int(s["len"])] = vals
            if int(s["flags"]) & 1:
                ao = int(s["aux_off"]) + r * int(s["aux_stride"])
                want_aux.view(np.uint16)[ao:ao + int(s["len"])] = bf16_rne_bits(vals)
            if int(s["flags"]) & 4:
                ao = int(s["aux_off"]) + r * int(s["aux_stride"])
                want_aux.view(b.dtype)[ao:ao + int(s["len"])] = vals
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), want)
    assert np.array_equal(aux.cpu().numpy(), want_aux)


def test_bf16_cast_rounding_special_values(gpu_device):
    """The fused cast rounds like torch's float -> bfloat16 (nearest-even, NaN -> 0x7FC0, inf kept)."""
    vals = np.array([0x3F800000, 0x3F808000, 0x3F818000, 0x3F80FFFF, 0x7F7FFFFF, 0x7F800000, 0xFF800000,
                     0x7FC00001, 0xFFFFFFFF, 0x80000000, 0x00000001, 0x807FFFFF, 0x3F7F7FFF, 0x3F7F8000,
                     0x477FE000, 0xC2F6E979], dtype=np.uint32)
    n = vals.size * 64
    host = np.tile(vals, 64)
    src = torch.from_numpy(host.view(np.int32)).to(gpu_device)
    dst = torch.zeros(n, dtype=torch.int32, device=gpu_device)
    aux = torch.zeros(n, dtype=torch.int16, device=gpu_device)
    t = np.zeros(2, dtype=SEGMENT_DTYPE)
    t[0] = (0, 0, 4, 1, 0, 0, n // 2, 1, 0, 0, 1, 0, 0, 0)           # vector path
    t[1] = (0, 0, 4, 1, n // 2, n // 2, n // 2 - 1, 1, 0, 0, 1, 0, n // 2 + 1, 0)  # element path
    plan = _native.Plan(t, [n * 4], [n * 4, n * 2])
    assert plan.stats().scalar_bytes > 0 and plan.stats().vector_bytes > 0
    plan.execute([src.data_ptr()], [dst.data_ptr(), aux.data_ptr()], torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = aux.cpu().numpy().view(np.uint16)
    want = np.concatenate([bf16_rne_bits(host[:n // 2]), [0], bf16_rne_bits(host[n // 2:n - 1])]).astype(np.uint16)
    got[n // 2] = 0
    assert np.array_equal(got, want)
    # Finite values and infinities round exactly as torch rounds them.  (torch's CPU kernels turn NaN
    # into 0xFFFF or 0x7FC0 depending on vectorisation; the cast here always gives 0x7FC0.)
    finite = (host & 0x7FFFFFFF) <= 0x7F800000
    torch_bf16 = torch.from_numpy(host.view(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(want[:n // 2][finite[:n // 2]], torch_bf16[:n // 2][finite[:n // 2]])
    assert (want[~np.concatenate([finite[:n // 2], [True], finite[n // 2:n - 1]])] == 0x7FC0).all()


@pytest.mark.parametrize("tuning", [{}, dict(chunk_index=False), dict(units=4), dict(persistent=True)])
def test_large_multichunk_plan(gpu_device, tuning):
    """More chunks than one grid row holds, 2-D segments with > 2^16 rows, segments split at 2^30
    units, and (persistent grid) many chunks per workgroup."""
    print(f"case large plan tuning {tuning}", flush=True)
    try:
        _native.set_tuning(**tuning)
        _large_multichunk_plan(gpu_device)
    finally:
        _native.set_tuning()


def _large_multichunk_plan(gpu_device):
    n = (1 << 26) + 12  # fp32 elements (256 MiB + 48 B)
    src = torch.arange(n, dtype=torch.int32, device=gpu_device)
    dst = torch.full((n,), -1, dtype=torch.int32, device=gpu_device)
    rows = [
        (0, 0, 4, 0, 0, 0, 1 << 24, 1, 0, 0, 0, 0, 0, 0),                      # contiguous 64 MiB
        (0, 0, 4, 0, 1 << 24, (1 << 24) + 4, 1000, 20000, 1000, 1004, 0, 0, 0, 0),  # strided, co-aligned
        (0, 0, 4, 0, 45_000_000, 45_000_001, 3_000_001, 1, 0, 0, 0, 0, 0, 0),  # misaligned by 4 bytes
        (0, 0, 1, 0, 200_000_001, 200_000_003, 8_000_000, 1, 0, 0, 0, 0, 0, 0),  # bytes, misaligned by 2
    ]
    t = np.zeros(len(rows), dtype=SEGMENT_DTYPE)
    t[:] = rows
    plan = _native.Plan(t, [n * 4], [n * 4], check_disjoint=True)
    st = plan.stats()
    assert st.payload_bytes == 4 * ((1 << 24) + 1000 * 20000 + 3_000_001) + 8_000_000
    assert st.n_chunks > 65536  # two rows of the one-workgroup-per-chunk grid
    plan.execute([src.data_ptr()], [dst.data_ptr()], torch.cuda.current_stream().cuda_stream)
    want = np.full(n, -1, dtype=np.int32)
    base = np.arange(n, dtype=np.int32)
    want[:1 << 24] = base[:1 << 24]
    for r in range(20000):
        so, do = (1 << 24) + r * 1000, (1 << 24) + 4 + r * 1004
        want[do:do + 1000] = base[so:so + 1000]
    want[45_000_001:48_000_002] = base[45_000_000:48_000_001]
    want.view(np.uint8)[200_000_003:208_000_003] = base.view(np.uint8)[200_000_001:208_000_001]
    assert np.array_equal(dst.cpu().numpy(), want)


def test_execute_errors(gpu_device):
    t = np.zeros(1, dtype=SEGMENT_DTYPE)
    t[0] = (0, 0, 4, 0, 0, 0, 16, 1, 0, 0, 0, 0, 0, 0)
    plan = _native.Plan(t, [1024], [1024])
    buf = torch.zeros(1024, dtype=torch.uint8, device=gpu_device)
    with pytest.raises(_native.EmrsError) as e:  # out of place only
        plan.execute([buf.data_ptr()], [buf.data_ptr() + 256], 0)
    assert e.value.code == -8
    other = torch.zeros(2048, dtype=torch.uint8, device=gpu_device)
    with pytest.raises(_native.EmrsError) as e:
        plan.execute([buf.data_ptr() + 4], [other.data_ptr()], 0)
    assert e.value.code == -3
    empty = _native.Plan(np.zeros(0, dtype=SEGMENT_DTYPE), [1024], [1024])
    empty.execute([buf.data_ptr()], [other.data_ptr()], 0)
    # A buffer no segment references may alias anything (a shared bf16 arena, say) or be NULL.
    buf.copy_((torch.arange(1024, device=gpu_device) % 251).to(torch.uint8))
    two = _native.Plan(t, [1024, 1024], [1024, 1024])
    two.execute([buf.data_ptr(), other.data_ptr()], [other.data_ptr() + 1024, other.data_ptr()], 0)
    two.execute([buf.data_ptr(), 0], [other.data_ptr() + 1024, 0], 0)
    torch.cuda.synchronize()
    assert torch.equal(other[1024:1088], buf[:64])


def test_destroy_right_after_execute(gpu_device):
    """A plan destroyed while its launch is still queued: the launch completes correctly."""
    n = 1 << 24
    src = torch.arange(n, dtype=torch.int32, device=gpu_device)
    dst = torch.zeros(n, dtype=torch.int32, device=gpu_device)
    side = torch.cuda.Stream(device=gpu_device)
    t = np.zeros(1, dtype=SEGMENT_DTYPE)
    t[0] = (0, 0, 4, 0, 0, 0, n, 1, 0, 0, 0, 0, 0, 0)
    for _ in range(3):
        dst.zero_()
        torch.cuda.synchronize()
        plan = _native.Plan(t, [n * 4], [n * 4])
        plan.execute([src.data_ptr()], [dst.data_ptr()], side.cuda_stream)
        plan.close()
        side.synchronize()
        assert torch.equal(dst, src)


def test_destroy_waits_only_for_its_own_launches(gpu_device):
    """Destroying a plan frees its tables after its own launches and does not wait for other work:
    a long queue of copies on another stream is still running when destroy returns."""
    n = 1 << 24
    src = torch.arange(n, dtype=torch.int32, device=gpu_device)
    dst = torch.zeros(n, dtype=torch.int32, device=gpu_device)
    big_a = torch.full((1 << 28,), 7, dtype=torch.int32, device=gpu_device)    # 1 GiB each
    big_b = torch.empty_like(big_a)
    side, other = torch.cuda.Stream(device=gpu_device), torch.cuda.Stream(device=gpu_device)
    t = np.zeros(1, dtype=SEGMENT_DTYPE)
    t[0] = (0, 0, 4, 0, 0, 0, n, 1, 0, 0, 0, 0, 0, 0)
    plan = _native.Plan(t, [n * 4], [n * 4])
    plan.execute([src.data_ptr()], [dst.data_ptr()], side.cuda_stream)    # uploads the tables
    torch.cuda.synchronize()
    dst.zero_()
    torch.cuda.synchronize()
    done = torch.cuda.Event()
    with torch.cuda.stream(other):
        for i in range(120):                     # about 40 ms of copies
            (big_b if i % 2 == 0 else big_a).copy_(big_a if i % 2 == 0 else big_b)
        done.record(other)
    plan.execute([src.data_ptr()], [dst.data_ptr()], side.cuda_stream)
    plan.close()
    assert not done.query(), "destroy waited for another stream's work"
    side.synchronize()
    assert torch.equal(dst, src)
    other.synchronize()
    assert bool((big_b == 7).all())


def test_manager_sequence(gpu_device):
    """ElasticMegatronManager.reshard through the tiny TP2DP4 -> TP1DP8 -> TP4DP2 sequence."""
    from elasticmegatron_amd import ElasticMegatronManager, tiny_llama2

    seq = [dict(world_size=8, tensor_model_parallel_size=2, pipeline_model_parallel_size=1),
           dict(world_size=8, tensor_model_parallel_size=1, pipeline_model_parallel_size=1),
           dict(world_size=8, tensor_model_parallel_size=4, pipeline_model_parallel_size=1)]
    mgr = ElasticMegatronManager(seq, tiny_llama2())
    mgr.training_state.fill_synthetic(SEED)
    for s in seq[1:]:
        st = mgr.reshard(new_parallel_strategy=s)
        bad, first = st.verify_synthetic(SEED)
        assert bad == 0, first
    # Back to the start: the round trip is the identity.
    st = mgr.reshard(new_parallel_strategy=seq[0])
    assert st.verify_synthetic(SEED)[0] == 0


def _random_cases():
    from tests.test_random_switches import _cases
    return _cases()


@pytest.mark.parametrize("spec,src,dst,bf16_source", _random_cases())
def test_random_switch_kernel_matches_oracle1(gpu_device, spec, src, dst, bf16_source):
    """The seeded random models and strategy pairs of tests/test_random_switches.py, on the GPU."""
    print(f"case {spec.name} {src} -> {dst} bf16 {bf16_source}", flush=True)
    space = build_virtual_model(spec)
    ls, ld = space.layout(src), space.layout(dst)
    a = TrainingState.allocate(ls, gpu_device)
    b = TrainingState.allocate(ld, gpu_device)
    a.fill_synthetic(SEED)
    for t in b.arenas():
        t.fill_(0) if t.dtype != torch.float32 else t.fill_(float("nan"))
    TransferManager(check_disjoint=True, bf16_source=bf16_source).transfer_optimizer_tensors(None, src=a, dst=b)
    got32, gotbf = extract(ld, _host_arenas(b))
    inv = model.inventory(spec)
    S, D = strat(src), strat(dst)
    dw, dbf, _ = oracle1.transfer(inv, spec, S, D, oracle1.build_src_world(inv, spec, S, SEED))
    assert compare(got32, gotbf, oracle1.flatten(dw), dbf) == []
