"""ctypes binding of libemrs (include/emrs.h).

The library is built in-tree by ``__graft_entry__.build()`` (or
``python -m elasticmegatron_amd.build``) into
``elasticmegatron_amd/csrc/libemrs.so``.  There is no fallback: when the
library is missing every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

from .resharding.layout import PIECE_DTYPE, SEGMENT_DTYPE

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "csrc", "libemrs.so")

EMRS_OK = 0
ERRORS = {
    -1: "EMRS_ERR_INVALID_ARGUMENT",
    -2: "EMRS_ERR_OUT_OF_BOUNDS",
    -3: "EMRS_ERR_MISALIGNED",
    -4: "EMRS_ERR_OVERLAP",
    -5: "EMRS_ERR_HIP",
    -6: "EMRS_ERR_NO_DEVICE",
    -7: "EMRS_ERR_TOO_MANY_BUFFERS",
    -8: "EMRS_ERR_ALIAS",
    -9: "EMRS_ERR_CAPTURE",
    -10: "EMRS_ERR_TOO_LARGE",
}
EMRS_PLAN_CHECK_DISJOINT = 1
EMRS_MAX_BUFFERS = 65535
EMRS_ARG_BUFFERS = 128  # buffers per side passed in kernel arguments (more use a device table)
EMRS_STATIC_SCRATCH_BYTES = 4 << 20  # device scratch of emrs_plan_compare_static

# Every function include/emrs.h declares.
EXPORTS = (
    "emrs_last_error", "emrs_abi_version", "emrs_device_count", "emrs_plan_create",
    "emrs_plan_stats_get", "emrs_plan_execute", "emrs_plan_destroy", "emrs_get_tuning",
    "emrs_set_tuning", "emrs_synth_fill", "emrs_synth_verify", "emrs_plan_compare", "emrs_xor_checksum",
    "emrs_plan_compare_static", "emrs_plan_prepare", "emrs_ipc_export", "emrs_ipc_open", "emrs_ipc_close",
    "emrs_ipc_open_count",
)

# struct emrs_compare_stats
COMPARE_DTYPE = np.dtype([("elements", "<u8"), ("mismatches", "<u8"), ("nonfinite", "<u8"), ("reserved", "<u8"),
                          ("sum_sq_diff", "<f8"), ("sum_sq_expected", "<f8"), ("max_abs_diff", "<f4"),
                          ("max_rel_diff", "<f4"), ("reserved2", "<u8")])


class EmrsError(RuntimeError):
    def __init__(self, code: int, where: str, msg: str):
        super().__init__(f"{where}: {ERRORS.get(code, code)}: {msg}")
        self.code = code


class PlanStats(ctypes.Structure):
    _fields_ = [
        ("n_segments", ctypes.c_uint64), ("n_device_segments", ctypes.c_uint64),
        ("payload_bytes", ctypes.c_uint64), ("read_bytes", ctypes.c_uint64), ("vector_bytes", ctypes.c_uint64),
        ("scalar_bytes", ctypes.c_uint64), ("n_chunks", ctypes.c_uint64),
        ("n_src_bufs", ctypes.c_uint32), ("n_dst_bufs", ctypes.c_uint32),
    ]


class Tuning(ctypes.Structure):
    _fields_ = [("blocks_per_cu", ctypes.c_uint32), ("nontemporal", ctypes.c_uint32),
                ("xcd_remap", ctypes.c_uint32), ("run", ctypes.c_uint32), ("persistent", ctypes.c_uint32),
                ("lanes", ctypes.c_uint32), ("units", ctypes.c_uint32), ("buffer_ops", ctypes.c_uint32),
                ("chunk_index", ctypes.c_uint32), ("warm_tables", ctypes.c_uint32)]


_lib: Optional[ctypes.CDLL] = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libemrs; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"libemrs is not built ({path} missing); run __graft_entry__.build() or "
            "python -m elasticmegatron_amd.build")
    lib = ctypes.CDLL(path)
    P, U64, U32, I = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int
    lib.emrs_last_error.restype = ctypes.c_char_p
    lib.emrs_last_error.argtypes = []
    lib.emrs_abi_version.restype = I
    lib.emrs_device_count.restype = I
    lib.emrs_plan_create.restype = I
    lib.emrs_plan_create.argtypes = [P, U64, P, U32, P, U32, U32, ctypes.POINTER(P)]
    lib.emrs_plan_stats_get.restype = I
    lib.emrs_plan_stats_get.argtypes = [P, ctypes.POINTER(PlanStats)]
    lib.emrs_plan_execute.restype = I
    lib.emrs_plan_execute.argtypes = [P, P, P, P]
    lib.emrs_plan_prepare.restype = I
    lib.emrs_plan_prepare.argtypes = [P, P]
    lib.emrs_plan_destroy.restype = I
    lib.emrs_plan_destroy.argtypes = [P]
    lib.emrs_get_tuning.restype = I
    lib.emrs_get_tuning.argtypes = [ctypes.POINTER(Tuning)]
    lib.emrs_set_tuning.restype = I
    lib.emrs_set_tuning.argtypes = [ctypes.POINTER(Tuning)]
    lib.emrs_synth_fill.restype = I
    lib.emrs_synth_fill.argtypes = [P, U64, P, P, U32, U64, P]
    lib.emrs_synth_verify.restype = I
    lib.emrs_synth_verify.argtypes = [P, U64, P, P, U32, U64, P, ctypes.POINTER(U64), ctypes.POINTER(U64)]
    lib.emrs_plan_compare.restype = I
    lib.emrs_plan_compare.argtypes = [P, P, P, P, P, U32, P, P]
    lib.emrs_plan_compare_static.restype = I
    lib.emrs_plan_compare_static.argtypes = [P, P, P, P, P, U32, P, P]
    lib.emrs_xor_checksum.restype = I
    lib.emrs_xor_checksum.argtypes = [P, U64, P, P]
    lib.emrs_ipc_export.restype = I
    lib.emrs_ipc_export.argtypes = [P, U64, P]
    lib.emrs_ipc_open.restype = I
    lib.emrs_ipc_open.argtypes = [P, ctypes.POINTER(P)]
    lib.emrs_ipc_close.restype = I
    lib.emrs_ipc_close.argtypes = [P]
    lib.emrs_ipc_open_count.restype = I
    lib.emrs_ipc_open_count.argtypes = []
    if lib.emrs_abi_version() != 8:
        raise RuntimeError("libemrs ABI version mismatch")
    _lib = lib
    return lib


def _check(rc: int, where: str) -> None:
    if rc != EMRS_OK:
        raise EmrsError(rc, where, load().emrs_last_error().decode(errors="replace"))


def _u64_buffer(vals: Sequence[int]) -> np.ndarray:
    a = np.array(vals if len(vals) else [0], dtype=np.uint64)
    if a.ndim != 1:
        raise ValueError("expected a flat sequence of integers")
    return a


def _ptr_array(ptrs: Sequence[int]):
    """A C array of device pointers over a numpy buffer (one conversion, no per-element ctypes
    objects: a per-tensor plan passes thousands).  The array keeps the buffer alive."""
    a = _u64_buffer(ptrs)
    return (ctypes.c_void_p * a.size).from_buffer(a)


def _u64_array(vals: Sequence[int]):
    a = _u64_buffer(vals)
    return (ctypes.c_uint64 * a.size).from_buffer(a)


def device_count() -> int:
    return int(load().emrs_device_count())


def get_tuning() -> Tuning:
    t = Tuning()
    _check(load().emrs_get_tuning(ctypes.byref(t)), "emrs_get_tuning")
    return t


def set_tuning(blocks_per_cu: int = 0, nontemporal: bool = True, xcd_remap: int = 1, run: int = 4,
               persistent: bool = False, lanes: int = 0, units: int = 1, buffer_ops: bool = False,
               chunk_index: bool = True, warm_tables: bool = True) -> None:
    """Launch shape of every later execution.  The default runs one workgroup of ``lanes`` lanes
    (0: 64) with ``units`` 16-byte units each (0: a whole chunk of 256 units per workgroup) per piece
    of a chunk, each finding its segment in the plan's chunk table (``chunk_index``; False: by a
    bounded binary search); ``persistent=True`` selects a persistent grid, which ``blocks_per_cu``
    and ``run`` shape.  ``xcd_remap`` gives each of the 8 XCDs one contiguous eighth of the chunks:
    1 (or True) in the persistent grid and for plans of at least 2^19 chunks, 2 always, 0 (or False)
    never.  ``warm_tables``: with the chunk table, a short kernel reads it and the segment
    descriptors just before each copy, so that a launch after unrelated work starts from cached
    tables."""
    t = Tuning(blocks_per_cu, 1 if nontemporal else 0, int(xcd_remap), run, 1 if persistent else 0, lanes,
               units, 1 if buffer_ops else 0, 1 if chunk_index else 0, 1 if warm_tables else 0)
    _check(load().emrs_set_tuning(ctypes.byref(t)), "emrs_set_tuning")


class Plan:
    """An uploaded-on-demand copy plan (emrs_plan)."""

    def __init__(self, segments: np.ndarray, src_buf_bytes: Sequence[int], dst_buf_bytes: Sequence[int],
                 check_disjoint: bool = False):
        lib = load()
        segs = np.ascontiguousarray(segments, dtype=SEGMENT_DTYPE)
        self._handle = ctypes.c_void_p()
        self.n_src = len(src_buf_bytes)
        self.n_dst = len(dst_buf_bytes)
        sb, db = _u64_array(src_buf_bytes), _u64_array(dst_buf_bytes)
        rc = lib.emrs_plan_create(segs.ctypes.data if len(segs) else None, len(segs), sb, self.n_src,
                                  db, self.n_dst, EMRS_PLAN_CHECK_DISJOINT if check_disjoint else 0,
                                  ctypes.byref(self._handle))
        _check(rc, "emrs_plan_create")

    def stats(self) -> PlanStats:
        st = PlanStats()
        _check(load().emrs_plan_stats_get(self._handle, ctypes.byref(st)), "emrs_plan_stats_get")
        return st

    def execute(self, src_ptrs: Sequence[int], dst_ptrs: Sequence[int], stream: int = 0) -> None:
        if len(src_ptrs) != self.n_src or len(dst_ptrs) != self.n_dst:
            raise ValueError("wrong number of base pointers")
        rc = load().emrs_plan_execute(self._handle, _ptr_array(src_ptrs), _ptr_array(dst_ptrs),
                                      ctypes.c_void_p(int(stream)))
        _check(rc, "emrs_plan_execute")

    def prepare(self, stream: int = 0) -> None:
        """Upload the plan's tables to the current device now (emrs_plan_prepare), so that its first
        execution there runs as fast as later ones."""
        _check(load().emrs_plan_prepare(self._handle, ctypes.c_void_p(int(stream))), "emrs_plan_prepare")

    def compare(self, src_ptrs: Sequence[int], dst_ptrs: Sequence[int], groups: Optional[np.ndarray] = None,
                aux_groups: Optional[np.ndarray] = None, n_groups: int = 1, stream: int = 0,
                no_alloc: bool = False) -> np.ndarray:
        """emrs_plan_compare: per group, how the destination differs from what the plan writes.

        ``groups`` / ``aux_groups`` hold one group id per input segment.
        Returns ``n_groups`` records of :data:`COMPARE_DTYPE`.  Waits for ``stream``.
        ``no_alloc``: run emrs_plan_compare_static, which allocates no device memory (its
        working set must fit in EMRS_STATIC_SCRATCH_BYTES).
        """
        if len(src_ptrs) != self.n_src or len(dst_ptrs) != self.n_dst:
            raise ValueError("wrong number of base pointers")
        n_in = self.stats().n_segments
        arrs = []
        for g in (groups, aux_groups):
            if g is None:
                arrs.append(None)
                continue
            g = np.ascontiguousarray(g, dtype=np.uint32)
            if g.shape != (n_in,):
                raise ValueError(f"need one group id per segment ({n_in})")
            arrs.append(g)
        out = np.zeros(max(1, n_groups), dtype=COMPARE_DTYPE)
        fn = load().emrs_plan_compare_static if no_alloc else load().emrs_plan_compare
        rc = fn(self._handle, _ptr_array(src_ptrs), _ptr_array(dst_ptrs),
                arrs[0].ctypes.data if arrs[0] is not None and n_in else None,
                arrs[1].ctypes.data if arrs[1] is not None and n_in else None,
                int(n_groups), out.ctypes.data, ctypes.c_void_p(int(stream)))
        _check(rc, "emrs_plan_compare_static" if no_alloc else "emrs_plan_compare")
        return out

    def close(self) -> None:
        if getattr(self, "_handle", None):
            load().emrs_plan_destroy(self._handle)
            self._handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def synth_fill(pieces: np.ndarray, ptrs: Sequence[int], buf_bytes: Sequence[int], seed: int, stream: int = 0) -> None:
    pcs = np.ascontiguousarray(pieces, dtype=PIECE_DTYPE)
    rc = load().emrs_synth_fill(pcs.ctypes.data if len(pcs) else None, len(pcs), _ptr_array(ptrs),
                                _u64_array(buf_bytes), len(ptrs), int(seed), ctypes.c_void_p(int(stream)))
    _check(rc, "emrs_synth_fill")


def xor_checksum(ptr: int, nbytes: int, out_ptr: int, stream: int = 0) -> None:
    """Enqueue the XOR of every 32-bit word of device memory [ptr, ptr + nbytes) into the device
    word at ``out_ptr``."""
    rc = load().emrs_xor_checksum(ctypes.c_void_p(int(ptr)), int(nbytes), ctypes.c_void_p(int(out_ptr)),
                                  ctypes.c_void_p(int(stream)))
    _check(rc, "emrs_xor_checksum")


def synth_verify(pieces: np.ndarray, ptrs: Sequence[int], buf_bytes: Sequence[int], seed: int,
                 stream: int = 0):
    """(mismatching elements, first bad (piece index, element index) or None)."""
    pcs = np.ascontiguousarray(pieces, dtype=PIECE_DTYPE)
    bad, first = ctypes.c_uint64(0), ctypes.c_uint64(0)
    rc = load().emrs_synth_verify(pcs.ctypes.data if len(pcs) else None, len(pcs), _ptr_array(ptrs),
                                  _u64_array(buf_bytes), len(ptrs), int(seed), ctypes.c_void_p(int(stream)),
                                  ctypes.byref(bad), ctypes.byref(first))
    _check(rc, "emrs_synth_verify")
    f = first.value
    return int(bad.value), (None if f == 2 ** 64 - 1 else (f >> 40, f & ((1 << 40) - 1)))


# struct emrs_ipc_buffer: an exported buffer, as plain bytes that travel between processes.
IPC_BUFFER_DTYPE = np.dtype([("handle", "u1", (64,)), ("offset", "<u8"), ("bytes", "<u8"),
                             ("allocation_bytes", "<u8"), ("device", "<i4"), ("reserved", "<u4")])
assert IPC_BUFFER_DTYPE.itemsize == 96
EMRS_IPC_MAX_ALLOCATION_BYTES = 2 << 30  # exclusive


def ipc_export(ptr: int, nbytes: int) -> np.ndarray:
    """emrs_ipc_export: the record describing device buffer [ptr, ptr + nbytes) to another process."""
    rec = np.zeros(1, dtype=IPC_BUFFER_DTYPE)
    _check(load().emrs_ipc_export(ctypes.c_void_p(int(ptr)), int(nbytes), rec.ctypes.data), "emrs_ipc_export")
    return rec[0]


def ipc_open(record) -> int:
    """emrs_ipc_open: map an exported buffer on the current device; returns its address."""
    rec = np.ascontiguousarray(np.asarray(record, dtype=IPC_BUFFER_DTYPE).reshape(1))
    out = ctypes.c_void_p()
    _check(load().emrs_ipc_open(rec.ctypes.data, ctypes.byref(out)), "emrs_ipc_open")
    return int(out.value)


def ipc_close(ptr: int) -> None:
    """emrs_ipc_close: drop one reference that :func:`ipc_open` returned."""
    _check(load().emrs_ipc_close(ctypes.c_void_p(int(ptr))), "emrs_ipc_close")


def ipc_open_count() -> int:
    """Allocations this process holds open through :func:`ipc_open`."""
    return int(load().emrs_ipc_open_count())
