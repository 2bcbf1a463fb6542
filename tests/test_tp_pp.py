"""TP send/recv maps (resharding_tp.py:94-191) and stage placement (resharding_pp.py:96-122).

Brute force: a full tensor is split into source TP shards the way Megatron
splits it (np.split along the partition dim; a fused SwiGLU fc1 holds
[W_t; V_t]); the maps, together with the SwiGLU shuffle/unshuffle, must
rebuild exactly the destination shards np.split gives.
"""

import numpy as np
import pytest

from elasticmegatron_amd.resharding.resharding_pp import LayerType, ParamPositionAttr
from elasticmegatron_amd.resharding.resharding_tp import TensorParallelAttr
from oracle import plan as oplan
from oracle.transfer import OptInfo

import torch


def _megatron_shards(x, T, dim, swiglu):
    if not swiglu:
        return np.split(x, T, axis=dim)
    w, v = np.split(x, 2, axis=0)
    return [np.concatenate([a, b]) for a, b in zip(np.split(w, T), np.split(v, T))]


def _run_maps(src_shards, send, recv, dst_shapes, swiglu, Ts, Td):
    """Apply send/recv maps with the SwiGLU shuffle as the reference's executor does."""
    src = [s.copy() for s in src_shards]
    if swiglu and Td > Ts:
        for s in range(Ts):
            info = OptInfo([torch.from_numpy(src[s].reshape(-1).astype(np.float32))] * 3, (0, src[s].size), src[s].shape)
            info.tensors = [info.tensors[0]]
            info.shuffle_swiglu(len(send[s]))
            src[s] = info.tensors[0].numpy().reshape(src[s].shape)
    dst = [np.full(shp, -1.0, dtype=np.float32) for shp in dst_shapes]
    for d in range(Td):
        for s, rng_d in recv[d].items():
            rng_s = send[s][d]
            sl_s = tuple(slice(*r) for r in (rng_s if isinstance(rng_s, tuple) else [(x.start, x.end) for x in rng_s.shapes]))
            sl_d = tuple(slice(*r) for r in (rng_d if isinstance(rng_d, tuple) else [(x.start, x.end) for x in rng_d.shapes]))
            dst[d][sl_d] = src[s][sl_s]
    if swiglu and Ts > Td:
        for d in range(Td):
            info = OptInfo([torch.from_numpy(dst[d].reshape(-1).copy())], (0, dst[d].size), dst[d].shape)
            info.unshuffle_swiglu(len(recv[d]))
            dst[d] = info.tensors[0].numpy().reshape(dst[d].shape)
    return dst


@pytest.mark.parametrize("shape,dim,swiglu", [((16, 8), 0, False), ((16, 8), 1, False), ((32, 8), 0, True),
                                              ((24,), 0, False)])
@pytest.mark.parametrize("Ts,Td", [(1, 4), (4, 1), (2, 4), (4, 2), (2, 2), (1, 1), (8, 2)])
def test_tp_maps_rebuild_np_split(shape, dim, swiglu, Ts, Td):
    if shape[dim] % max(Ts, Td) or (swiglu and (shape[0] // 2) % max(Ts, Td)):
        pytest.skip("shape not divisible")
    x = np.arange(int(np.prod(shape)), dtype=np.float32).reshape(shape)
    src = _megatron_shards(x, Ts, dim, swiglu)
    want = _megatron_shards(x, Td, dim, swiglu)
    attr = TensorParallelAttr(shape, True, dim)
    info = attr.reshard(Ts, Td)
    got = _run_maps(src, info.send_info, info.recv_info, [w.shape for w in want], swiglu, Ts, Td)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)
    p = dict(shape=shape, tp=True, pdim=dim, swiglu=swiglu, expert=None)
    osend, orecv = oplan.tp_maps(p, Ts, Td)
    got = _run_maps(src, osend, orecv, [w.shape for w in want], swiglu, Ts, Td)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)
    # The product's maps and the oracle's are the same maps.
    conv = lambda m: {a: {b: tuple((r.start, r.end) for r in pr.shapes) for b, pr in v.items()} for a, v in m.items()}
    assert conv(info.send_info) == osend and conv(info.recv_info) == orecv


def test_non_tp_param_sent_by_tp_rank0_to_all():
    attr = TensorParallelAttr((512,), False, -1)
    info = attr.reshard(2, 4)
    assert list(info.send_info) == [0] and sorted(info.send_info[0]) == [0, 1, 2, 3]
    assert all(list(m) == [0] for m in info.recv_info.values())
    with pytest.raises(AssertionError):
        attr.reshard(3, 4)


@pytest.mark.parametrize("pp", [1, 2, 4, 8])
def test_stage_ids(pp):
    L = 32
    mk = lambda lt, **kw: ParamPositionAttr(lt, L, **kw)
    assert mk(LayerType.WORD_EMBEDDING).get_model_param_stage_id(pp) == 0
    assert mk(LayerType.FINAL_LAYERNORM).get_model_param_stage_id(pp) == pp - 1
    assert mk(LayerType.OUTPUT_LAYER).get_model_param_stage_id(pp) == pp - 1
    assert mk(LayerType.OUTPUT_LAYER, shared_embedding=True).get_model_param_stage_id(pp) == (-1 if pp == 1 else pp - 1)
    per = L // pp
    for l in range(L):
        sid = mk(LayerType.TRANSFORMER_LAYER, transformer_layer_id=l).get_model_param_stage_id(pp)
        assert sid == l // per
        assert oplan.stage(dict(where="layer", layer=l, shared=False), pp, L) == sid
    info = mk(LayerType.TRANSFORMER_LAYER, transformer_layer_id=17).reshard(2, 4)
    assert (info.src_pp_rank, info.dst_pp_rank) == (1, 2)
