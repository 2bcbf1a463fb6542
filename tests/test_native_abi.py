"""The C ABI: the library loads, exports what include/emrs.h declares, and
validates plans on the host (no GPU needed)."""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

from elasticmegatron_amd import _native
from elasticmegatron_amd.resharding.layout import PIECE_DTYPE, SEGMENT_DTYPE

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "emrs.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+char\s*\*\s*|int\s+)(emrs_\w+)\s*\(", text, re.M)))


def test_exports_every_declared_symbol():
    lib = _native.load()
    declared = _declared()
    assert set(declared) == set(_native.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.emrs_abi_version() == 8


def test_record_layouts_match_header():
    class Seg(ctypes.Structure):
        _fields_ = [(n, ctypes.c_uint32) for n in ("src_buf", "dst_buf", "elem_bytes", "flags")] + \
                   [(n, ctypes.c_uint64) for n in ("src_off", "dst_off", "len", "rows", "src_stride", "dst_stride")] + \
                   [("aux_buf", ctypes.c_uint32), ("reserved", ctypes.c_uint32), ("aux_off", ctypes.c_uint64),
                    ("aux_stride", ctypes.c_uint64)]

    assert ctypes.sizeof(Seg) == SEGMENT_DTYPE.itemsize == 88
    for name, (dt, off) in SEGMENT_DTYPE.fields.items():
        assert getattr(Seg, name).offset == off
    assert PIECE_DTYPE.itemsize == 88

    class Cmp(ctypes.Structure):  # struct emrs_compare_stats
        _fields_ = [(n, ctypes.c_uint64) for n in ("elements", "mismatches", "nonfinite", "reserved")] + \
                   [("sum_sq_diff", ctypes.c_double), ("sum_sq_expected", ctypes.c_double),
                    ("max_abs_diff", ctypes.c_float), ("max_rel_diff", ctypes.c_float), ("reserved2", ctypes.c_uint64)]

    assert ctypes.sizeof(Cmp) == _native.COMPARE_DTYPE.itemsize == 64
    for name, (dt, off) in _native.COMPARE_DTYPE.fields.items():
        assert getattr(Cmp, name).offset == off


def _seg(**kw):
    row = dict(src_buf=0, dst_buf=0, elem_bytes=4, flags=0, src_off=0, dst_off=0, len=16, rows=1,
               src_stride=0, dst_stride=0, aux_buf=0, reserved=0, aux_off=0, aux_stride=0)
    row.update(kw)
    t = np.zeros(1, dtype=SEGMENT_DTYPE)
    for k, v in row.items():
        t[0][k] = v
    return t


@pytest.mark.parametrize("kw,code", [
    (dict(elem_bytes=3), -1),
    (dict(rows=0), -1),
    (dict(dst_buf=1), -1),
    (dict(rows=2, len=16, src_stride=16, dst_stride=8), -1),
    (dict(src_off=250, len=16), -2),
    (dict(dst_off=1, len=256), -2),
    (dict(rows=3, len=10, src_stride=200, dst_stride=10), -2),
    (dict(flags=8), -1),
    (dict(flags=5, aux_off=64), -1),                      # bf16 image and duplicate together
    (dict(flags=4, aux_buf=1), -1),
    (dict(flags=4, aux_off=250, len=16), -2),             # duplicate extent in 4-byte elements
    (dict(flags=4, elem_bytes=8, aux_off=121, len=8), -2),  # ... and in 8-byte elements
    (dict(flags=4, rows=2, src_stride=16, dst_stride=16, aux_stride=8), -1),
    (dict(flags=2, src_buf=1), -1),
    (dict(flags=2, dst_off=1000, len=16), -2),
    (dict(reserved=1), -1),
    (dict(flags=1, elem_bytes=2), -1),
    (dict(flags=1, aux_buf=1), -1),
    (dict(flags=1, aux_off=500, len=16), -2),
    (dict(flags=1, rows=2, src_stride=16, dst_stride=16, aux_stride=8), -1),
])
def test_plan_create_rejects(kw, code):
    with pytest.raises(_native.EmrsError) as e:
        _native.Plan(_seg(**kw), [1024], [1024])
    assert e.value.code == code


def test_plan_create_overlap_check():
    t = np.concatenate([_seg(dst_off=0, len=10), _seg(src_off=20, dst_off=9, len=4)])
    _native.Plan(t, [1024], [1024])  # allowed without the check
    with pytest.raises(_native.EmrsError) as e:
        _native.Plan(t, [1024], [1024], check_disjoint=True)
    assert e.value.code == -4
    # bf16 images count as destination writes too.
    t = np.concatenate([_seg(dst_off=0, len=8, flags=1, aux_buf=1, aux_off=0), _seg(dst_off=16, len=8, flags=1,
                                                                                   aux_buf=1, aux_off=4)])
    with pytest.raises(_native.EmrsError) as e:
        _native.Plan(t, [1024], [1024, 1024], check_disjoint=True)
    assert e.value.code == -4
    # So do duplicates, over elem_bytes-wide elements: the duplicate's bytes [128, 192) meet the second
    # row's destination bytes [160, 192).
    _native.Plan(_seg(dst_off=0, len=8, flags=4, aux_off=64), [1024], [1024], check_disjoint=True)
    t = np.concatenate([_seg(dst_off=0, len=8, flags=4, aux_off=16, elem_bytes=8),
                        _seg(src_off=0, dst_off=20, len=4, elem_bytes=8)])
    with pytest.raises(_native.EmrsError) as e:
        _native.Plan(t, [1024], [1024], check_disjoint=True)
    assert e.value.code == -4
    t = np.concatenate([_seg(dst_off=0, len=8, flags=4, aux_off=4), _seg(dst_off=16, len=8)])
    with pytest.raises(_native.EmrsError) as e:
        _native.Plan(t, [1024], [1024], check_disjoint=True)  # duplicate meets its own destination
    assert e.value.code == -4


def test_too_many_buffers():
    with pytest.raises(_native.EmrsError) as e:
        _native.Plan(_seg(), [64] * 65536, [64])
    assert e.value.code == -7


def test_plan_stats_classify_alignment():
    z = (0, 0, 0, 0)
    rows = [
        (0, 0, 4, 0, 0, 0, 64, 1, 0, 0) + z,      # vector: 256 bytes
        (0, 0, 4, 0, 1, 1, 12, 1, 0, 0) + z,      # co-aligned, 4 B off: 3 head + 8 body + 1 tail elements
        (0, 0, 4, 0, 1, 2, 8, 1, 0, 0) + z,       # not co-aligned: scalar
        (0, 0, 2, 0, 0, 0, 8, 4, 16, 8) + z,      # strided bf16 rows of 16 bytes: vector
        (0, 0, 2, 0, 0, 64, 3, 4, 8, 5) + z,      # strided, odd: scalar
        (0, 0, 4, 1, 256, 256, 32, 1, 0, 0, 1, 0, 8, 0),   # cast, aux 8-byte aligned: vector
        (0, 0, 4, 1, 320, 320, 32, 1, 0, 0, 1, 0, 50, 0),  # cast, aux 4 bytes off: scalar
    ]
    t = np.zeros(len(rows), dtype=SEGMENT_DTYPE)
    t[:] = rows
    st = _native.Plan(t, [4096], [4096, 4096]).stats()
    assert st.read_bytes == 256 + 48 + 32 + 64 + 24 + 128 + 128
    assert st.payload_bytes == st.read_bytes + 64 + 64
    assert st.vector_bytes == 256 + 32 + 64 + 128
    assert st.scalar_bytes == 16 + 32 + 24 + 128
    assert st.n_segments == 7


def test_zero_fill_reads_nothing():
    """EMRS_SEG_ZERO_FILL: the source offset is ignored and no source byte is counted as read."""
    rows = [
        (0, 0, 4, 2, 10 ** 12, 0, 64, 1, 0, 0, 0, 0, 0, 0),        # zeros, vector path
        (0, 0, 4, 3, 0, 100, 16, 2, 0, 20, 1, 0, 4, 24),           # zeros + bf16 zeros, 2-D
        (0, 0, 2, 2, 0, 1000, 5, 1, 0, 0, 0, 0, 0, 0),             # 2-byte zeros, scalar path
        (0, 0, 4, 0, 0, 200, 8, 1, 0, 0, 0, 0, 0, 0),              # an ordinary copy
    ]
    t = np.zeros(len(rows), dtype=SEGMENT_DTYPE)
    t[:] = rows
    st = _native.Plan(t, [64], [4096, 4096], check_disjoint=True).stats()
    assert st.read_bytes == 32
    assert st.payload_bytes == 256 + 128 + 64 + 10 + 32
    assert st.n_segments == 4


def test_empty_plan_and_no_device_errors():
    plan = _native.Plan(np.zeros(0, dtype=SEGMENT_DTYPE), [16], [16])
    assert plan.stats().payload_bytes == 0
    plan.prepare(0)  # nothing to upload: no device needed
    if _native.device_count() == 0:
        # Host-side checks happen before any device work; a real execution needs a GPU.
        t = _native.Plan(_seg(), [1024], [1024])
        with pytest.raises(_native.EmrsError) as e:
            t.execute([0x10000], [0x20000], 0)
        assert e.value.code == -6
        with pytest.raises(_native.EmrsError) as e:
            t.prepare(0)
        assert e.value.code == -6


def _two_seg_plan(n_bufs=2):
    t = np.zeros(2, dtype=SEGMENT_DTYPE)
    t[0] = (0, 0, 4, 0, 0, 0, 16, 1, 0, 0, 0, 0, 0, 0)
    t[1] = (n_bufs - 1, n_bufs - 1, 4, 0, 0, 0, 16, 1, 0, 0, 0, 0, 0, 0)
    return _native.Plan(t, [1024] * n_bufs, [1024] * n_bufs)


@pytest.mark.parametrize("n_bufs", [2, 300])   # kernel-argument path and device-table path
def test_alias_checks_before_any_device_work(n_bufs):
    """Host-side buffer checks of emrs_plan_execute: out of place, destinations disjoint."""
    plan = _two_seg_plan(n_bufs)
    base = 1 << 40
    src = [base + i * 4096 for i in range(n_bufs)]
    dst = [base + (1 << 30) + i * 4096 for i in range(n_bufs)]
    # Two referenced destinations overlapping.
    bad = list(dst)
    bad[n_bufs - 1] = dst[0] + 512
    with pytest.raises(_native.EmrsError) as e:
        plan.execute(src, bad, 0)
    assert e.value.code == -8
    # A referenced source overlapping a referenced destination.
    bad = list(src)
    bad[0] = dst[n_bufs - 1] + 16
    with pytest.raises(_native.EmrsError) as e:
        plan.execute(bad, dst, 0)
    assert e.value.code == -8
    # Sources may overlap each other, unreferenced buffers may alias anything or be NULL;
    # the call then gets as far as looking for a device.
    ok_src = list(src)
    ok_src[n_bufs - 1] = src[0] + 16
    ok_dst = list(dst)
    if n_bufs > 2:
        ok_dst[1] = dst[0]
        ok_src[1] = 0
    if torch.cuda.is_available():
        return
    with pytest.raises(_native.EmrsError) as e:
        plan.execute(ok_src, ok_dst, 0)
    assert e.value.code == -6
    # Misaligned referenced base.
    bad = list(src)
    bad[0] += 8
    with pytest.raises(_native.EmrsError) as e:
        plan.execute(bad, dst, 0)
    assert e.value.code == -3


@pytest.mark.parametrize("n_bufs", [2, 300])
def test_compare_accepts_overlapping_buffers(n_bufs):
    """A comparison only reads: a destination overlapping a source (a state that took over part of
    its source's memory) passes its base checks, where an execution refuses it."""
    plan = _two_seg_plan(n_bufs)
    base = 1 << 40
    src = [base + i * 4096 for i in range(n_bufs)]
    dst = list(src)                      # every destination is its source's memory
    with pytest.raises(_native.EmrsError) as e:
        plan.execute(src, dst, 0)
    assert e.value.code == -8
    if torch.cuda.is_available():
        return
    with pytest.raises(_native.EmrsError) as e:
        plan.compare(src, dst)
    assert e.value.code == -6            # got as far as looking for a device
    bad = list(dst)
    bad[0] += 8
    with pytest.raises(_native.EmrsError) as e:
        plan.compare(src, bad)
    assert e.value.code == -3            # alignment is still checked


def test_xor_checksum_rejects_bad_arguments_before_touching_a_device():
    with pytest.raises(_native.EmrsError) as e:
        _native.xor_checksum(0x1000, 16, 0)               # no output word
    assert e.value.code == -1
    with pytest.raises(_native.EmrsError) as e:
        _native.xor_checksum(0, 16, 0x2000)               # no buffer
    assert e.value.code == -1
    for ptr, n in ((0x1008, 16), (0x1000, 24)):            # 16-byte alignment of address and size
        with pytest.raises(_native.EmrsError) as e:
            _native.xor_checksum(ptr, n, 0x2000)
        assert e.value.code == -3


def test_tuning_defaults_and_rejections():
    """emrs_tuning: the default launch shape reads back, settings round-trip, and values outside the
    documented ranges are refused without changing the current setting (no device needed)."""
    assert ctypes.sizeof(_native.Tuning) == 40  # ten uint32 fields, as in emrs.h
    t = _native.get_tuning()
    assert (t.persistent, t.lanes, t.units, t.nontemporal, t.run, t.chunk_index, t.warm_tables) == \
        (0, 64, 1, 1, 4, 1, 1)
    try:
        _native.set_tuning(warm_tables=False)
        assert _native.get_tuning().warm_tables == 0
        _native.set_tuning(lanes=128, units=0, persistent=True, run=7, blocks_per_cu=3, chunk_index=False)
        t = _native.get_tuning()
        assert (t.persistent, t.lanes, t.run, t.blocks_per_cu, t.chunk_index) == (1, 128, 7, 3, 0)
        assert _native.get_tuning().units == 2   # 0: one chunk of 256 units per workgroup
        _native.set_tuning(lanes=64, units=1, buffer_ops=True)
        assert (_native.get_tuning().lanes, _native.get_tuning().units, _native.get_tuning().buffer_ops) == (64, 1, 1)
        for x in (0, 2, 1):
            _native.set_tuning(xcd_remap=x)
            assert _native.get_tuning().xcd_remap == x
        _native.set_tuning(lanes=128, persistent=True, run=7, blocks_per_cu=3)
        for kw in (dict(lanes=96), dict(lanes=512), dict(run=(1 << 20) + 1), dict(blocks_per_cu=65),
                   dict(units=3), dict(units=8), dict(lanes=128, units=4), dict(lanes=256, units=2),
                   dict(xcd_remap=3)):
            with pytest.raises(_native.EmrsError) as e:
                _native.set_tuning(**kw)
            assert e.value.code == -1
            assert _native.get_tuning().lanes == 128  # unchanged
        _native.set_tuning(lanes=0)  # 0 selects the default lane count
        assert _native.get_tuning().lanes == 64
    finally:
        _native.set_tuning()
    t = _native.get_tuning()
    assert (t.persistent, t.lanes, t.units, t.run, t.blocks_per_cu, t.xcd_remap, t.chunk_index, t.warm_tables) == \
        (0, 64, 1, 4, 0, 1, 1, 1)
