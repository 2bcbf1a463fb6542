"""Tensor-parallel resharding info of one parameter.

Mirrors ``TensorParallelAttr`` / ``TensorParallelReshardingInfo`` of the
reference (elastic_megatron/resharding/resharding_tp.py:11-208).  Ranges are
in TP-local coordinates, exactly as the reference builds them:

* scale-up by k (``src < dst``): src TP rank s sends chunk i of its local
  tensor (split along ``partition_dim``) to dst TP rank ``s*k + i``, which
  receives it into its whole local tensor (resharding_tp.py:157-175);
* scale-down by k: dst TP rank d receives src TP rank ``d*k + i`` into chunk i
  of its local tensor (resharding_tp.py:177-191);
* a parameter that is not tensor-parallel is sent whole by src TP rank 0 to
  every dst TP rank (resharding_tp.py:119-139).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Sequence, Tuple

from .util import ParamRange


@dataclass
class TensorParallelReshardingInfo:
    # src_tp_rank -> {dst_tp_rank: range in the src rank's local tensor}
    send_info: Dict[int, Dict[int, ParamRange]]
    # dst_tp_rank -> {src_tp_rank: range in the dst rank's local tensor}
    recv_info: Dict[int, Dict[int, ParamRange]]


def is_pow2(n: int) -> bool:
    return n >= 1 and (n & (n - 1)) == 0


class TensorParallelAttr:
    """TP attributes of a parameter given by its full (TP=1) shape."""

    def __init__(self, full_shape: Sequence[int], tensor_model_parallel: bool = False,
                 partition_dim: int = -1, partition_stride: int = 1):
        if partition_stride != 1:
            raise AssertionError("Only support partition_stride==1")  # resharding_tp.py:50
        self.tensor_model_parallel = bool(tensor_model_parallel)
        self.partition_dim = partition_dim if tensor_model_parallel else -1
        if self.tensor_model_parallel and not (0 <= partition_dim < len(full_shape)):
            raise AssertionError("tensor-parallel parameter needs a valid partition_dim")
        self.partition_stride = partition_stride
        self.model_param_range_in_group = ParamRange(param_shape=tuple(full_shape))
        self._ranges: Dict[int, ParamRange] = {1: self.model_param_range_in_group}
        self._cache: Dict[Tuple[int, int], TensorParallelReshardingInfo] = {}

    @property
    def full_shape(self) -> Tuple[int, ...]:
        return self.model_param_range_in_group.to_shape()

    def get_model_param_range(self, parallel_group_size: int) -> ParamRange:
        """Local range of TP rank 0 at the given TP size (resharding_tp.py:76-92)."""
        if parallel_group_size == 1 or not self.tensor_model_parallel:
            return self.model_param_range_in_group
        r = self._ranges.get(parallel_group_size)
        if r is None:
            r = self.model_param_range_in_group.chunk(parallel_group_size, self.partition_dim)[0]
            self._ranges[parallel_group_size] = r
        return r

    def local_shape(self, parallel_group_size: int) -> Tuple[int, ...]:
        return self.get_model_param_range(parallel_group_size).to_shape()

    def reshard(self, src_size: int, dst_size: int) -> TensorParallelReshardingInfo:
        assert is_pow2(src_size) and is_pow2(dst_size), "TP sizes must be powers of two"
        key = (src_size, dst_size)
        info = self._cache.get(key)
        if info is None:
            if not self.tensor_model_parallel:
                info = self._without_split(src_size, dst_size)
            else:
                info = self._with_split(src_size, dst_size)
            self._cache[key] = info
        return info

    def _without_split(self, src_size: int, dst_size: int) -> TensorParallelReshardingInfo:
        whole = self.get_model_param_range(src_size)
        send = {0: {d: whole for d in range(dst_size)}}
        recv = {d: {0: whole} for d in range(dst_size)}
        return TensorParallelReshardingInfo(send_info=send, recv_info=recv)

    def _with_split(self, src_size: int, dst_size: int) -> TensorParallelReshardingInfo:
        src_range = self.get_model_param_range(src_size)
        dst_range = self.get_model_param_range(dst_size)
        send: Dict[int, Dict[int, ParamRange]] = {}
        recv: Dict[int, Dict[int, ParamRange]] = {}
        if src_size < dst_size:
            k = dst_size // src_size
            chunks: List[ParamRange] = src_range.chunk(k, self.partition_dim)
            for s in range(src_size):
                for i, c in enumerate(chunks):
                    send.setdefault(s, {})[s * k + i] = c
                    recv[s * k + i] = {s: chunks[0]}
            return TensorParallelReshardingInfo(send_info=send, recv_info=recv)
        k = src_size // dst_size
        chunks = dst_range.chunk(k, self.partition_dim)
        for d in range(dst_size):
            for i, c in enumerate(chunks):
                recv.setdefault(d, {})[d * k + i] = c
                send[d * k + i] = {d: chunks[0]}
        return TensorParallelReshardingInfo(send_info=send, recv_info=recv)

    def _key(self):
        return (self.tensor_model_parallel, self.partition_dim, self.partition_stride,
                self.model_param_range_in_group)

    def __hash__(self):
        return hash(self._key())

    def __eq__(self, other):
        # Equal attributes, not equal hashes: two attributes whose hashes collide stay distinct.
        return isinstance(other, TensorParallelAttr) and self._key() == other._key()

    def __str__(self):
        split = f"split on dim {self.partition_dim}" if self.tensor_model_parallel else "replicated"
        return f"<TP {split}, full {'x'.join(map(str, self.full_shape))}>"
