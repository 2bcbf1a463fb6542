"""GPU: the executor at the limits of its ABI.

- 128 source and destination buffers (passed in kernel arguments) and 3000
  (passed through a device table of pointers) in one plan.
- Segments beyond 2^30 units, which emrs_plan_create splits so that the
  kernel's unit arithmetic stays in 32 bits: a 1-D and a 2-D byte segment
  of 1.5 GiB each (the element-wise path, where a unit is one byte).
- 70,000 segments in one plan, with and without the chunk table.
Expected results come from torch slicing on the device.
"""

import numpy as np
import pytest
import torch

from elasticmegatron_amd import _native
from elasticmegatron_amd.resharding.layout import SEGMENT_DTYPE

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [_native.EMRS_ARG_BUFFERS, 3000])
def test_many_buffers(gpu_device, n):
    """128 buffers per side (kernel arguments) and 3000 (device pointer table)."""
    size = 4096
    srcs = []
    for i in range(n):
        t = torch.arange(size, device=gpu_device, dtype=torch.int32).to(torch.uint8) ^ (i % 251)
        srcs.append(t)
    dsts = [torch.zeros(size, dtype=torch.uint8, device=gpu_device) for _ in range(n)]
    rows = []
    for i in range(n):
        j = n - 1 - i
        k = i % 200
        rows.append((i, j, 1, 0, k, 3 * k, 1000 + k, 1, 0, 0, 0, 0, 0, 0))        # element-wise path
        rows.append((i, j, 4, 0, 512, 768, 64, 1, 0, 0, 0, 0, 0, 0))             # 16-byte path
    t = np.zeros(len(rows), dtype=SEGMENT_DTYPE)
    t[:] = rows
    plan = _native.Plan(t, [size] * n, [size] * n, check_disjoint=True)
    plan.execute([s.data_ptr() for s in srcs], [d.data_ptr() for d in dsts], torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for i in range(n):
        j, k = n - 1 - i, i % 200
        want = torch.zeros(size, dtype=torch.uint8, device=gpu_device)
        want[3 * k:3 * k + 1000 + k] = srcs[i][k:k + 1000 + k]
        want[768 * 4:(768 + 64) * 4] = srcs[i][512 * 4:(512 + 64) * 4]
        assert torch.equal(dsts[j], want), (i, j)


def test_pointer_table_reuse_and_new_bases(gpu_device):
    """A plan over more than 128 buffers keeps the pointer table of its first execution and reuses it
    while the bases repeat; other bases get a table of their own.  Every call must land where its
    own bases say, on the current stream and on a second one."""
    n, size = 300, 1024
    rng = np.random.default_rng(7)
    srcs = [torch.from_numpy(rng.integers(0, 256, size, dtype=np.uint8)).to(gpu_device) for _ in range(n)]
    sets = [[torch.zeros(size, dtype=torch.uint8, device=gpu_device) for _ in range(n)] for _ in range(2)]
    t = np.zeros(n, dtype=SEGMENT_DTYPE)
    t[:] = [(i, (i * 7) % n, 4, 0, 16, 32, 128, 1, 0, 0, 0, 0, 0, 0) for i in range(n)]
    plan = _native.Plan(t, [size] * n, [size] * n, check_disjoint=True)
    side = torch.cuda.Stream()
    sp = [s.data_ptr() for s in srcs]
    for k, (which, stream) in enumerate([(0, None), (0, None), (1, None), (0, side), (1, side), (0, None)]):
        print(f"case pointer table call {k}: destination set {which}", flush=True)
        for d in sets[which]:
            d.zero_()
        st = stream if stream is not None else torch.cuda.current_stream()
        st.wait_stream(torch.cuda.current_stream())
        plan.execute(sp, [d.data_ptr() for d in sets[which]], st.cuda_stream)
        torch.cuda.synchronize()
        for i in range(n):
            got = sets[which][(i * 7) % n]
            assert torch.equal(got[128:640], srcs[i][64:576]), (k, i)
            assert int(got[:128].sum()) == 0 and int(got[640:].sum()) == 0, (k, i)


def _kind_table(rng, n, size):
    """Segment i: source buffer i -> destination buffer i, second destination (cast image or
    duplicate) in destination buffer n + i.  Kinds cycle: copy (every element width, aligned or
    not, 1-D or strided), zero fill, fp32 with its bf16 image, duplicate."""
    rows = []
    for i in range(n):
        kind = i % 4
        eb = 4 if kind == 2 else int(rng.choice([1, 2, 4, 8]))
        ln = int(rng.integers(1, 60))  # the largest extent, 3 rows of 8-byte elements, fits in 4 KB
        r = int(rng.choice([1, 1, 3]))
        ss = ds = 0
        if r > 1:
            ss, ds = ln + int(rng.integers(0, 9)), ln + int(rng.integers(0, 9))
        if rng.random() < 0.5:  # 16-byte friendly
            unit = 16 // eb
            ln = (ln // unit + 1) * unit
            if r > 1:
                ss, ds = 2 * ln, 2 * ln
        nb = size // eb
        so = int(rng.integers(0, nb - ((r - 1) * ss + ln)))
        do = int(rng.integers(0, nb - ((r - 1) * ds + ln)))
        if rng.random() < 0.5:
            so, do = so - so % (16 // eb), do - do % (16 // eb)
        flags, ao, astr = 0, 0, 0
        if kind == 1:
            flags = 2
        elif kind == 2:
            flags, ao, astr = 1, do, ds
        elif kind == 3:
            flags, ao, astr = 4, do, ds
        rows.append((i, i, eb, flags, so, do, ln, r, ss, ds, n + i if kind in (2, 3) else 0, 0, ao, astr))
    t = np.zeros(n, dtype=SEGMENT_DTYPE)
    t[:] = rows
    return t


def _expected(t, srcs_h, n, size):
    from tests.helpers import bf16_rne_bits

    out = [np.zeros(size, dtype=np.uint8) for _ in range(2 * n)]
    for s in t:
        eb, i = int(s["elem_bytes"]), int(s["src_buf"])
        dt = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[eb]
        a, b, x = srcs_h[i].view(dt), out[i].view(dt), out[n + i]
        for r in range(int(s["rows"])):
            so = int(s["src_off"]) + r * int(s["src_stride"])
            do = int(s["dst_off"]) + r * int(s["dst_stride"])
            vals = np.zeros(int(s["len"]), dtype=dt) if int(s["flags"]) & 2 else a[so:so + int(s["len"])]
            b[do:do + int(s["len"])] = vals
            ao = int(s["aux_off"]) + r * int(s["aux_stride"])
            if int(s["flags"]) & 1:
                x.view(np.uint16)[ao:ao + int(s["len"])] = bf16_rne_bits(vals)
            if int(s["flags"]) & 4:
                x.view(dt)[ao:ao + int(s["len"])] = vals
    return out


@pytest.mark.parametrize("lanes,buffer_ops", [(64, False), (256, False), (64, True), (128, False)])
def test_table_bases_every_segment_kind(gpu_device, lanes, buffer_ops):
    """A plan over 200 source and 400 destination buffers, with every kind of segment, run on the
    bases of its first call (the segment table resolved against them, no base lookup in the
    kernel), on other bases (the pointer table), and on the first bases again."""
    n, size = 200, 4096
    rng = np.random.default_rng(11)
    srcs_h = [rng.integers(0, 256, size, dtype=np.uint8) for _ in range(n)]
    srcs = [torch.from_numpy(h).to(gpu_device) for h in srcs_h]
    sets = [[torch.zeros(size, dtype=torch.uint8, device=gpu_device) for _ in range(2 * n)] for _ in range(2)]
    t = _kind_table(rng, n, size)
    plan = _native.Plan(t, [size] * n, [size] * (2 * n), check_disjoint=True)
    want = _expected(t, srcs_h, n, size)
    sp = [s.data_ptr() for s in srcs]
    try:
        _native.set_tuning(lanes=lanes, buffer_ops=buffer_ops)
        for k, which in enumerate([0, 0, 1, 0, 1]):
            print(f"case table bases lanes {lanes} buffer {buffer_ops} call {k}: destination set {which}",
                  flush=True)
            for d in sets[which]:
                d.zero_()
            plan.execute(sp, [d.data_ptr() for d in sets[which]], torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            for j in range(2 * n):
                assert np.array_equal(sets[which][j].cpu().numpy(), want[j]), (k, j)
    finally:
        _native.set_tuning()


def test_segments_beyond_two_to_the_thirty_units(gpu_device):
    nbytes = 3 << 29  # 1.5 GiB
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=gpu_device)
    dst = torch.zeros(nbytes + 64, dtype=torch.uint8, device=gpu_device)
    n1 = nbytes - 3
    t = np.zeros(1, dtype=SEGMENT_DTYPE)
    t[0] = (0, 0, 1, 0, 1, 2, n1, 1, 0, 0, 0, 0, 0, 0)  # offsets 1 and 2: element-wise, 1-byte units
    plan = _native.Plan(t, [nbytes], [nbytes + 64])
    assert plan.stats().n_device_segments >= 2 and plan.stats().scalar_bytes == n1
    plan.execute([src.data_ptr()], [dst.data_ptr()], torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(dst[2:2 + n1], src[1:1 + n1])
    assert int(dst[:2].sum()) == 0 and int(dst[2 + n1:].sum()) == 0

    # 2-D: 1,500,000 rows of 1,000 bytes with strides 1,001 and 1,003 (split by rows).
    rows, ln = 1_500_000, 1000
    del dst
    src2 = src[:rows * 1001]
    t[0] = (0, 0, 1, 0, 0, 5, ln, rows, 1001, 1003, 0, 0, 0, 0)
    need = 5 + rows * 1003  # whole last row stride, so that the result can be viewed as rows x 1003
    dst2 = torch.zeros(need, dtype=torch.uint8, device=gpu_device)
    plan = _native.Plan(t, [rows * 1001], [need])
    assert plan.stats().n_device_segments >= 2
    plan.execute([src2.data_ptr()], [dst2.data_ptr()], torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = dst2[5:5 + rows * 1003].view(rows, 1003)[:, :ln]
    want = src2.view(rows, 1001)[:, :ln]
    assert torch.equal(got, want)
    assert int(dst2[5:5 + rows * 1003].view(rows, 1003)[:, ln:].sum()) == 0


@pytest.mark.parametrize("buffer_ops", [False, True])
def test_long_row_pitches_are_emitted_row_by_row(gpu_device, buffer_ops):
    """Row pitches of 2^23 bytes and more (here 8 MiB and 12 MiB) are emitted one row at a time, so
    the buffer-instruction path's 32-bit offsets cover every piece; the copy is unchanged."""
    rows, n = 5, 1000
    ps, pd = (1 << 21), (3 << 20)          # fp32 elements: 8 MiB and 12 MiB pitches
    src = torch.randint(0, 1 << 30, (rows * ps,), dtype=torch.int32, device=gpu_device)
    dst = torch.zeros(rows * pd, dtype=torch.int32, device=gpu_device)
    t = np.zeros(2, dtype=SEGMENT_DTYPE)
    t[0] = (0, 0, 4, 0, 8, 4, n, rows, ps, pd, 0, 0, 0, 0)          # long pitches: split by rows
    t[1] = (0, 0, 4, 0, 8 + n, 4 + n, 16, 4, 64, 64, 0, 0, 0, 0)    # short pitches: one device segment
    plan = _native.Plan(t, [rows * ps * 4], [rows * pd * 4], check_disjoint=True)
    assert plan.stats().n_device_segments >= rows + 1
    try:
        _native.set_tuning(buffer_ops=buffer_ops)
        print(f"case long pitches buffer {buffer_ops}", flush=True)
        plan.execute([src.data_ptr()], [dst.data_ptr()], torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
    finally:
        _native.set_tuning()
    want = torch.zeros_like(dst)
    for r in range(rows):
        want[4 + r * pd:4 + r * pd + n] = src[8 + r * ps:8 + r * ps + n]
    for r in range(4):
        want[4 + n + r * 64:4 + n + r * 64 + 16] = src[8 + n + r * 64:8 + n + r * 64 + 16]
    assert torch.equal(dst, want)


@pytest.mark.parametrize("chunk_index", [True, False])
def test_more_than_65535_segments(gpu_device, chunk_index):
    """70,000 one-chunk segments in a random order, every seventh a zero fill: more segments than
    one grid row of the device-side chunk-table build, which then strides over them."""
    n, unit = 70_000, 1024  # fp32 elements per segment: one 4 KB chunk
    g = torch.Generator().manual_seed(7)
    perm = torch.randperm(n, generator=g)
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (n * unit,), dtype=torch.int32, generator=g).to(gpu_device)
    dst = torch.full((n * unit,), -1, dtype=torch.int32, device=gpu_device)
    t = np.zeros(n, dtype=SEGMENT_DTYPE)
    t["elem_bytes"] = 4
    t["src_off"] = perm.numpy().astype(np.uint64) * unit
    t["dst_off"] = np.arange(n, dtype=np.uint64) * unit
    t["len"] = unit
    t["rows"] = 1
    zero = np.arange(n) % 7 == 3
    t["flags"][zero] = 2
    plan = _native.Plan(t, [n * unit * 4], [n * unit * 4])
    assert plan.stats().n_device_segments >= n
    print(f"case {n} segments, chunk_index={chunk_index}", flush=True)
    try:
        _native.set_tuning(chunk_index=chunk_index)
        plan.execute([src.data_ptr()], [dst.data_ptr()], torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
    finally:
        _native.set_tuning()
    want = src.view(n, unit)[perm.to(gpu_device)].clone()
    want[torch.from_numpy(zero).to(gpu_device)] = 0
    assert torch.equal(dst.view(n, unit), want)
