"""Inter-process hand-off of a training state on one machine.

Replaces elastic_megatron/transfer/ipc_manager.py.  There, the old process
packs a CUDA-IPC handle for the storage of every optimizer tensor of every
parameter (``_make_cuda_tensor_info``, :23-51), sends the pickled payload over
a ZMQ socket and exits (``send_training_state``, :54-132); the new process
rebuilds one tensor per handle (``receive_training_state``, :135-155), clones
them into the optimizer of a model it built on the meta device and only then
reshards (tools/agent/env_utils.py:326-483, the swap at :423-433).

Here the old process holds its whole state in a :class:`SharedTrainingState`:
the four arenas of a layout, each cut into granules of less than 2 GiB, one
device allocation per granule, because device memory is shared one
allocation at a time and only below that size.  ``send_training_state``
exports every granule once (a few dozen handles for a 7B model instead of one
per tensor) and writes a JSON payload: the model, the strategy, the granule
size and the handle records.  ``receive_training_state`` maps the granules in
the new process; the reshard then runs straight from the mapped memory into
the new process's own state, one copy-plan launch re-based onto the granules
(:class:`~..resharding.granules.GranuleBuffers`), with no clone.  The
transport (a pipe, a socket, a file) is the caller's: the payload is one line
of text, and holds nothing that runs when it is read.

The memory stays owned by the old process, which must keep it until the new
process has closed its mappings: :func:`notify_release` /
:func:`wait_for_release` carry that signal over the same kind of channel.
"""

from __future__ import annotations

import dataclasses
import json
from typing import IO, Callable, Dict, List, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from .. import _native
from ..megatron_manager.parallel_strategy import ParallelStrategy
from ..resharding.granules import DEFAULT_GRANULE_BYTES, GranuleBuffers
from ..resharding.layout import ARENA_NAMES, ARENA_PARAM, StrategyLayout, split_vocab_rows
from ..resharding.model_spec import ModelSpec

PAYLOAD_FORMAT = "emrs-shared-state/1"
RELEASED = "released"
FREED = "freed"
_STRATEGY_FIELDS = ("world_size", "tensor_model_parallel_size", "pipeline_model_parallel_size",
                    "context_parallel_size", "num_distributed_optimizer_instances", "expert_model_parallel_size",
                    "expert_tensor_parallel_size", "sequence_parallel")
_DTYPES = (torch.float32, torch.float32, torch.float32, torch.bfloat16)


class SharedTrainingState:
    """Every rank's state of one strategy, held in granules that another process can map.

    The same state as :class:`~..megatron_manager.training_state.TrainingState`
    (fp32 ``main`` / ``exp_avg`` / ``exp_avg_sq`` of every rank, bf16 params of
    every model-parallel shard), stored as ``buffers`` (arena granules in
    buffer order).  Owned: the granules are torch tensors of this process.
    Imported: they are another process's memory, mapped by
    :func:`receive_training_state`, and :meth:`close` unmaps them.
    """

    def __init__(self, layout: StrategyLayout, buffers: GranuleBuffers, ptrs: Sequence[int],
                 device: torch.device, tensors: Optional[List[torch.Tensor]] = None):
        if len(ptrs) != len(buffers):
            raise ValueError("one pointer per granule")
        self.layout = layout
        self.buffers = buffers
        self._ptrs = list(ptrs)
        self._device = torch.device(device)
        self.tensors = tensors          # owned granules; None when imported
        self._open = tensors is None    # imported mappings not yet closed
        self._released = [False] * 4    # per arena: freed (owned) or unmapped (imported)
        self._handed_over = set()       # owned granules now held by another state (hand_over)
        # Imported states: called with an arena's index once its mappings are closed, so that the
        # exporting process can free that arena (see :func:`release_hook`).
        self.on_release: Optional[Callable[[int], None]] = None

    # ----- construction -----
    @classmethod
    def allocate(cls, layout: StrategyLayout, device=None, granule_bytes: int = DEFAULT_GRANULE_BYTES,
                 param_granules: Optional[List[torch.Tensor]] = None,
                 adopted: Optional[Sequence[Sequence[torch.Tensor]]] = None,
                 kinds: Tuple[int, ...] = (0, 1, 2)) -> "SharedTrainingState":
        """Uninitialised granules for ``layout``, one allocation each; ``param_granules`` may be the
        bf16 granules of another state of the same model-parallel layout, shared instead.
        ``adopted``: per fp32 arena (main, exp_avg, exp_avg_sq), the same number of granules of
        another state to hold as this state's leading granules of that arena instead of allocating
        them (a Group-ZeRO switch that leaves instance 0 in place; the other state then hands them
        over, see :meth:`hand_over`).  ``kinds``: the fp32 arenas whose granules are allocated now;
        the others start without memory and are allocated with :meth:`allocate_kind`, as a staged
        switch does."""
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        if adopted is not None and tuple(kinds) != (0, 1, 2):
            raise ValueError("a state that takes over granules allocates every fp32 arena at once")
        if dev.type != "cuda":
            raise RuntimeError("a shared state lives in GPU memory")
        bufs = GranuleBuffers(layout, granule_bytes)
        keep = list(bufs.granules_of(ARENA_PARAM))
        if param_granules is not None and [t.numel() for t in param_granules] != [bufs.numel[b] for b in keep]:
            raise ValueError("the shared param granules do not match the layout")
        held = {}
        if adopted is not None:
            if len(adopted) != 3 or len({len(ts) for ts in adopted}) != 1:
                raise ValueError("adopted takes the same number of granules for each fp32 arena")
            for a, ts in enumerate(adopted):
                ids = bufs.granules_of(a)
                if len(ts) > len(ids):
                    raise ValueError("more adopted granules than the arena has")
                for j, t in enumerate(ts):
                    b = ids[j]
                    if t.dtype != torch.float32 or t.numel() != bufs.numel[b] or t.device != dev \
                            or not t.is_contiguous():
                        raise ValueError(f"adopted granule {j} of {ARENA_NAMES[a]} does not match the layout")
                    held[b] = t
        tensors = []
        for b, (a, n) in enumerate(zip(bufs.arena, bufs.numel)):
            if a == ARENA_PARAM and param_granules is not None:
                tensors.append(param_granules[b - keep[0]])
            elif b in held:
                tensors.append(held[b])
            elif a == ARENA_PARAM or a in kinds:
                tensors.append(torch.empty(n, dtype=_DTYPES[a], device=dev))
            else:
                tensors.append(None)
        st = cls(layout, bufs, [0 if t is None else t.data_ptr() for t in tensors], dev, tensors)
        for a in range(3):
            st._released[a] = a not in kinds
        return st

    def allocate_kind(self, kind: int) -> None:
        """Allocate the granules of fp32 arena ``kind`` (0 main, 1 exp_avg, 2 exp_avg_sq) if it has
        none: a staged switch allocates each destination arena just before its stage.  With the
        source in granules of the same size, those are the granules its previous stage released,
        straight from torch's cache."""
        if self.imported:
            raise RuntimeError("an imported state's granules belong to the exporting process")
        if kind not in (0, 1, 2):
            raise ValueError("allocate_kind takes an fp32 arena: 0 main, 1 exp_avg, 2 exp_avg_sq")
        if not self._released[kind]:
            return
        for b in self.buffers.granules_of(kind):
            t = torch.empty(self.buffers.numel[b], dtype=torch.float32, device=self._device)
            self.tensors[b] = t
            self._ptrs[b] = t.data_ptr()
            self._handed_over.discard(b)
        self._released[kind] = False

    def leading_fp32_granules(self, n: int) -> List[List[torch.Tensor]]:
        """The first ``n`` granules of every fp32 arena of an owned state, for another state to
        adopt (``allocate(..., adopted=...)``)."""
        if self.imported:
            raise RuntimeError("an imported state's granules belong to the exporting process")
        out = []
        for a in range(3):
            ids = self.buffers.granules_of(a)
            if n > len(ids) or self._released[a] or any(b in self._handed_over for b in ids[:n]):
                raise ValueError(f"{ARENA_NAMES[a]} has no {n} leading granules to give")
            out.append([self.tensors[b] for b in ids[:n]])
        return out

    def hand_over(self, n: int) -> None:
        """Forget the first ``n`` granules of every fp32 arena: another state adopted them and
        owns them from now on.  Releasing this state then leaves them alone, and its pointers to
        them read 0."""
        if self.imported:
            raise RuntimeError("an imported state's granules belong to the exporting process")
        for a in range(3):
            ids = self.buffers.granules_of(a)
            if n > len(ids):
                raise ValueError(f"{ARENA_NAMES[a]} has only {len(ids)} granules")
            for b in ids[:n]:
                self._handed_over.add(b)
                self.tensors[b] = None
                self._ptrs[b] = 0

    # ----- what the transfer manager reads -----
    @property
    def parallel_strategy(self) -> ParallelStrategy:
        return self.layout.strategy

    @property
    def device(self) -> torch.device:
        return self._device

    @property
    def granule_bytes(self) -> int:
        return self.buffers.granule_bytes

    @property
    def imported(self) -> bool:
        return self.tensors is None

    def buffer_ptrs(self) -> List[int]:
        """Base pointer of every granule; 0 for the granules of a released arena and for those
        handed over to another state."""
        if self.imported and not self._open:
            raise RuntimeError("the shared state's mappings are closed")
        return [0 if self._released[a] else p for a, p in zip(self.buffers.arena, self._ptrs)]

    def buffer_bytes(self) -> List[int]:
        """Bytes of every granule; 0 for the granules of a released arena and for those handed
        over to another state."""
        nb = self.buffers.nbytes()
        return [0 if self._released[a] or b in self._handed_over else n
                for b, (a, n) in enumerate(zip(self.buffers.arena, nb))]

    # ----- lifetime -----
    def release_kind(self, kind: int) -> None:
        """Release fp32 arena ``kind`` (0 main, 1 exp_avg, 2 exp_avg_sq), as a staged switch does
        once that arena is copied (the reference releases each optimizer tensor once it is sent,
        resharding_metadata.py:58-65).  Owned granules are freed.  An imported state's granules of
        that arena are unmapped (after the device has finished with them), then ``on_release`` is
        called so that the exporting process can free them."""
        if kind not in (0, 1, 2):
            raise ValueError("release_kind takes an fp32 arena: 0 main, 1 exp_avg, 2 exp_avg_sq")
        if self._released[kind]:
            return
        if not self.imported:
            for b in self.buffers.granules_of(kind):
                if b not in self._handed_over and self.tensors[b] is not None:
                    self.tensors[b].untyped_storage().resize_(0)
            self._released[kind] = True
            return
        if not self._open:
            return
        self._unmap(self.buffers.granules_of(kind))
        self._released[kind] = True
        if self.on_release is not None:
            self.on_release(kind)

    def release_optimizer(self) -> None:
        """Drop the fp32 state (training_state.py:313-315): owned granules are freed, and an
        imported state is unmapped whole (its bf16 params went to the new state with the switch)."""
        if self.imported:
            self.close()
            return
        for a in range(3):
            self.release_kind(a)

    def _unmap(self, granules) -> None:
        with torch.cuda.device(self._device):
            torch.cuda.synchronize(self._device)
            for b in granules:
                _native.ipc_close(self._ptrs[b])

    def close(self) -> None:
        """Unmap every granule of an imported state still mapped (emrs_ipc_close).  Waits for the
        device first, so work that still reads the mappings has finished."""
        if not self.imported or not self._open:
            return
        self._unmap([b for b, a in enumerate(self.buffers.arena) if not self._released[a]])
        self._open = False
        self._released = [True] * 4

    # ----- synthetic workload -----
    _SYNTH_MAX_BUFFERS = 128   # buffers per emrs_synth_fill / emrs_synth_verify call

    def _per_arena(self, pieces: np.ndarray):
        """The pieces of each arena in batches of at most 128 granules, addressed by granule within
        the batch: (arena, pieces, granule pointers, granule bytes, first granule's buffer id).  A
        released or handed-over granule has no bytes, so a piece there is refused before any launch."""
        pcs = self.buffers.split_pieces(pieces)
        ptrs, nbytes = self.buffer_ptrs(), self.buffer_bytes()
        for a in range(4):
            ids = self.buffers.granules_of(a)
            for lo in range(ids.start, ids.stop, self._SYNTH_MAX_BUFFERS):
                hi = min(lo + self._SYNTH_MAX_BUFFERS, ids.stop)
                sel = pcs[(pcs["buf"] >= lo) & (pcs["buf"] < hi)].copy()
                if len(sel) == 0:
                    continue
                sel["buf"] -= lo
                yield a, sel, ptrs[lo:hi], nbytes[lo:hi], lo

    def fill_synthetic(self, seed: int, params=None, fp32: bool = True, bf16: bool = True) -> None:
        """Write the seeded synthetic values of every stored element (see csrc/synth.hip)."""
        st = torch.cuda.current_stream(self._device).cuda_stream
        with torch.cuda.device(self._device):
            for _, pcs, ptrs, nb, _ in self._per_arena(self.layout.pieces(params, include_bf16=bf16,
                                                                           include_fp32=fp32)):
                _native.synth_fill(pcs, ptrs, nb, seed, st)

    def verify_synthetic(self, seed: int, params=None, fp32: bool = True, bf16: bool = True,
                         vocab_rows: Optional[int] = None) -> Tuple[int, Optional[dict]]:
        """(mismatching elements, first bad element) against the seeded synthetic values."""
        pcs = self.layout.pieces(params, include_bf16=bf16, include_fp32=fp32)
        if vocab_rows is not None:
            pcs, zero = split_vocab_rows(self.layout, pcs, vocab_rows)
            if zero:
                raise NotImplementedError("re-padded vocabularies are checked on a TrainingState")
        st = torch.cuda.current_stream(self._device).cuda_stream
        bad, first = 0, None
        with torch.cuda.device(self._device):
            for a, sel, ptrs, nb, lo in self._per_arena(pcs):
                n, f = _native.synth_verify(sel, ptrs, nb, seed, st)
                bad += n
                if f is not None and first is None:
                    p = sel[f[0]]
                    first = dict(arena=ARENA_NAMES[a], param_id=int(p["param_id"]), kind=int(p["kind"]),
                                 element=int(f[1]), granule=lo + int(p["buf"]))
        return bad, first

    # ----- export -----
    def export(self) -> List[np.ndarray]:
        """One emrs_ipc_buffer record per granule (ipc_manager.py:23-51)."""
        if self.imported:
            raise RuntimeError("an imported state is exported by the process that owns it")
        if any(self._released) or self._handed_over:
            raise RuntimeError("part of this state is released or handed over to another state: only a whole "
                               "state can be exported")
        with torch.cuda.device(self._device):
            return [_native.ipc_export(p, n) for p, n in zip(self._ptrs, self.buffers.nbytes())]


def strategy_to_dict(s: ParallelStrategy) -> Dict:
    return {k: getattr(s, k) for k in _STRATEGY_FIELDS}


def _record_hex(rec) -> str:
    return np.asarray(rec, dtype=_native.IPC_BUFFER_DTYPE).reshape(1).tobytes().hex()


def _record_of(text: str) -> np.ndarray:
    raw = bytes.fromhex(text)
    if len(raw) != _native.IPC_BUFFER_DTYPE.itemsize:
        raise ValueError("malformed buffer record")
    return np.frombuffer(raw, dtype=_native.IPC_BUFFER_DTYPE)[0]


def send_training_state(state: SharedTrainingState, wfile: Optional[IO[str]] = None,
                        misc: Optional[Dict] = None) -> Dict:
    """Export ``state`` for another process (ipc_manager.py:54-132).

    Waits for the work queued on the state's device, so the exported memory
    holds its final values, then returns the payload: the model, the
    strategy, the granule size, one handle record per granule, and ``misc``
    (any JSON-serialisable values the caller carries along, as the reference
    carries its iteration, RNG and scheduler state).  With ``wfile`` it is
    also written there as one line of JSON, flushed.  The caller keeps the
    state alive until the importer has released it (:func:`wait_for_release`).
    """
    with torch.cuda.device(state.device):
        torch.cuda.synchronize(state.device)
    payload = {
        "format": PAYLOAD_FORMAT,
        "model_spec": dataclasses.asdict(state.layout.space.spec),
        "strategy": strategy_to_dict(state.parallel_strategy),
        "granule_bytes": state.granule_bytes,
        "buffers": [{"key": list(k), "record": _record_hex(r)} for k, r in zip(state.buffers.keys, state.export())],
        "misc": misc or {},
    }
    if wfile is not None:
        wfile.write(json.dumps(payload) + "\n")
        wfile.flush()
    return payload


def receive_training_state(source: Union[Dict, IO[str], str], device=None, space=None
                           ) -> Tuple[SharedTrainingState, Dict]:
    """Map an exported state into this process (ipc_manager.py:135-155); returns (state, misc).

    ``source`` is the payload, its JSON text, or a file to read one line of
    it from.  ``space``: the virtual model to lay the state out in (one is
    built from the payload's model when None; it must describe the same
    model).  The layout is rebuilt from the model and the strategy, and every
    granule's size is checked against it before anything is mapped.
    """
    if isinstance(source, dict):
        payload = source
    else:
        text = source if isinstance(source, str) else source.readline()
        if not text:
            raise EOFError("no payload: the exporting process sent nothing")
        payload = json.loads(text)
    if payload.get("format") != PAYLOAD_FORMAT:
        raise ValueError(f"not a shared training state payload: {payload.get('format')!r}")
    from ..resharding.virtual_param import build_virtual_model

    spec = ModelSpec(**payload["model_spec"])
    if space is None:
        space = build_virtual_model(spec)
    elif space.spec != spec:
        raise ValueError("the payload describes another model than the given virtual model")
    strategy = ParallelStrategy(**payload["strategy"])
    layout = space.layout(strategy)
    bufs = GranuleBuffers(layout, payload["granule_bytes"])
    recs = [_record_of(b["record"]) for b in payload["buffers"]]
    if [tuple(b["key"]) for b in payload["buffers"]] != [tuple(k) for k in bufs.keys] or \
            [int(r["bytes"]) for r in recs] != bufs.nbytes():
        raise ValueError("the payload's granules do not match the layout rebuilt from its model and strategy")
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    ptrs: List[int] = []
    with torch.cuda.device(dev):
        try:
            for r in recs:
                ptrs.append(_native.ipc_open(r))
        except Exception:
            for p in ptrs:
                _native.ipc_close(p)
            raise
    return SharedTrainingState(layout, bufs, ptrs, dev), payload.get("misc", {})


def notify_release(wfile: IO[str], arena: Optional[str] = None) -> None:
    """Tell the exporting process that this process has closed its mappings: all of them, or with
    ``arena`` those of that arena only (a staged switch releases the source arena by arena)."""
    wfile.write((RELEASED if arena is None else f"{RELEASED} {arena}") + "\n")
    wfile.flush()


def wait_for_release(rfile: IO[str], on_arena: Optional[Callable[[str], None]] = None) -> bool:
    """Block until the importer's release notice (True) or the end of the channel (False).
    ``on_arena(name)`` is called for each fp32 arena the importer releases before that."""
    while True:
        line = rfile.readline()
        if not line:
            return False
        words = line.split()
        if words == [RELEASED]:
            return True
        if len(words) == 2 and words[0] == RELEASED and words[1] in ARENA_NAMES[:3] and on_arena is not None:
            on_arena(words[1])


def notify_freed(wfile: IO[str], arena: str) -> None:
    """The exporter's answer to an arena's release notice: its memory is back with the driver."""
    wfile.write(f"{FREED} {arena}\n")
    wfile.flush()


def wait_for_freed(rfile: IO[str], arena: str) -> bool:
    """Block until the exporter has freed ``arena`` (True) or the channel ends (False)."""
    while True:
        line = rfile.readline()
        if not line:
            return False
        if line.split() == [FREED, arena]:
            return True


def release_hook(wfile: IO[str], rfile: IO[str]) -> Callable[[int], None]:
    """``SharedTrainingState.on_release`` for a received state: tells the exporter over ``wfile``
    that an arena's mappings are closed and waits on ``rfile`` until it has freed that arena, so
    that the next stage of a staged switch can allocate in its place."""
    def release(arena: int) -> None:
        name = ARENA_NAMES[arena]
        notify_release(wfile, name)
        if not wait_for_freed(rfile, name):
            raise RuntimeError(f"the exporting process ended before it freed {name}")
    return release
