"""Verification of a reshard (emrs_plan_compare), on the CPU.

The numpy model of emrs_plan_compare (tests.helpers.compare_numpy) is pinned
here against the reference's checkpoint check restated with torch
(tools/ckpt/compare_ckpt.py:52-66: max |A - B|, max |A - B| / (|B| + 1e-12),
RMS, relative RMS), per parameter and tensor kind, on states with planted
differences.  The grouped lowering that labels every element with its
parameter must write exactly what the executed lowering writes.
"""

import numpy as np
import pytest
import torch

from elasticmegatron_amd import _native
from elasticmegatron_amd.megatron_manager.parallel_strategy import ParallelStrategy as PS
from elasticmegatron_amd.resharding.layout import ARENA_PARAM
from elasticmegatron_amd.resharding.lowering import lower_redundant_backup, lower_transfer
from elasticmegatron_amd.resharding.virtual_param import build_virtual_model
from elasticmegatron_amd.transfer.verify import KIND_NAMES, TensorDiff, VerifyReport, report_from_stats
from tests.helpers import (SEED, SMALL_CASES, compare_numpy, execute_numpy, new_arenas, piece_fill_numpy,
                           small_llama2, small_llama3)


def _switches():
    for name, factory, seq in SMALL_CASES:
        a, b = seq[0], seq[1]
        yield pytest.param(factory, a, b, id=name)


@pytest.mark.parametrize("factory,src,dst", list(_switches()))
@pytest.mark.parametrize("bf16_source", ["cast", "copy"])
def test_grouped_lowering_writes_the_same(factory, src, dst, bf16_source):
    space = build_virtual_model(factory())
    ls, ld = space.layout(src), space.layout(dst)
    table = lower_transfer(ls, ld, bf16_source=bf16_source)
    gt, groups, aux_groups = lower_transfer(ls, ld, bf16_source=bf16_source, with_groups=True)
    assert len(groups) == len(aux_groups) == len(gt)
    a = new_arenas(ls)
    piece_fill_numpy(ls.pieces(), a, SEED)
    b1, b2 = new_arenas(ld), new_arenas(ld)
    execute_numpy(table, a, b1)
    execute_numpy(gt, a, b2)
    for x, y in zip(b1, b2):
        assert np.array_equal(x, y)
    # Every row of every segment lies inside the holders of its group's parameter and kind (holders of
    # one parameter on consecutive ranks can be adjacent, so they are merged first).
    holders = {}
    for vp in space.all_virtual_params:
        if not ld.has_param(vp):
            continue
        for h in ld.fp32_holders(vp):
            for k in (1, 2, 3):
                holders.setdefault((4 * vp.global_index + k, k - 1), []).append((h.offset, h.offset + h.hi - h.lo))
        for h in ld.bf16_holders(vp):
            holders.setdefault((4 * vp.global_index, ARENA_PARAM), []).append((h.offset, h.offset + h.hi - h.lo))
    merged = {}
    for key, ivs in holders.items():
        out = []
        for b0, b1 in sorted(ivs):
            if out and b0 <= out[-1][1]:
                out[-1][1] = max(out[-1][1], b1)
            else:
                out.append([b0, b1])
        merged[key] = out

    def inside(key, lo, n):
        return any(b0 <= lo and lo + n <= b1 for b0, b1 in merged.get(key, []))

    for s, g, ga in zip(gt, groups, aux_groups):
        n = int(s["len"])
        for r in range(int(s["rows"])):
            assert inside((int(g), int(s["dst_buf"])), int(s["dst_off"]) + r * int(s["dst_stride"]), n)
            if int(s["flags"]) & 1:
                assert inside((int(ga), ARENA_PARAM), int(s["aux_off"]) + r * int(s["aux_stride"]), n)


def _plant(arenas, rng, n):
    """Change n random elements of each destination arena (fp32 and bf16 bits); returns the count per arena."""
    specials = np.array([0x7FC00000, 0x7F800000, 0xFF800000, 0x80000000], dtype=np.uint32)
    out = []
    for i, arr in enumerate(arenas):
        idx = rng.choice(arr.size, size=n, replace=False)
        if arr.dtype == np.uint32:
            new = arr[idx] ^ (np.uint32(1) << rng.integers(0, 31, n).astype(np.uint32))
            new[:4] = specials  # NaN, +inf, -inf, -0
        else:
            new = arr[idx] ^ (np.uint16(1) << rng.integers(0, 15, n).astype(np.uint16))
        changed = int((new != arr[idx]).sum())
        arr[idx] = new
        out.append(changed)
    return out


@pytest.mark.parametrize("factory,src,dst,kind", [
    (small_llama3, PS(8, 2, 2), PS(8, 4, 1), "transfer"),
    (small_llama2, PS(6, 1, 1), PS(12, 1, 1, num_distributed_optimizer_instances=2), "backup_up"),
])
def test_compare_model_equals_compare_ckpt(factory, src, dst, kind):
    """compare_numpy's per-tensor figures equal compare_ckpt.py's formulas on the same tensors."""
    space = build_virtual_model(factory())
    ls, ld = space.layout(src), space.layout(dst)
    if kind == "transfer":
        table, groups, aux_groups = lower_transfer(ls, ld, with_groups=True)
    else:
        table, groups, aux_groups = lower_redundant_backup(ls, ld, scale_up=True, with_groups=True)
    a = new_arenas(ls)
    piece_fill_numpy(ls.pieces(), a, SEED)
    want = new_arenas(ld, fill=0)
    execute_numpy(table, a, want)
    got = [x.copy() for x in want]
    if kind != "transfer":
        got[ARENA_PARAM] = want[ARENA_PARAM]  # the bf16 arena is not part of a Group-ZeRO switch
    planted = _plant(got[:3] if kind != "transfer" else got, np.random.default_rng(0), 64)
    n_groups = 4 * len(space.all_virtual_params)
    stats = compare_numpy(table, groups, aux_groups, n_groups, a, got)
    assert int(stats["mismatches"].sum()) <= sum(planted)
    report = report_from_stats(stats, [p.name for p in space.all_virtual_params])

    # The same figures from compare_ckpt.py's formulas, per (parameter, kind), on fp32 tensors.
    for vp in space.all_virtual_params:
        if not ld.has_param(vp):
            continue
        for k in range(4):
            if k == 0:
                hs = [(ARENA_PARAM, h) for h in ld.bf16_holders(vp)] if kind == "transfer" else []
            else:
                hs = [(k - 1, h) for h in ld.fp32_holders(vp)]
            if not hs:
                continue

            def cat(arenas):
                parts = [arenas[b][h.offset:h.offset + h.hi - h.lo] for b, h in hs]
                x = np.concatenate(parts)
                x = (x.astype(np.uint32) << 16).view(np.float32) if x.dtype == np.uint16 else x.view(np.float32)
                return torch.from_numpy(x.copy())

            va, vb = cat(got), cat(want)
            t = report.tensors[(vp.name, KIND_NAMES[k])]
            assert t.elements == va.numel()
            bits = torch.from_numpy(np.concatenate([got[b][h.offset:h.offset + h.hi - h.lo] for b, h in hs]).astype(
                np.int64)) != torch.from_numpy(np.concatenate(
                    [want[b][h.offset:h.offset + h.hi - h.lo] for b, h in hs]).astype(np.int64))
            assert t.mismatches == int(bits.sum())
            diff = (va - vb).abs()
            fin = torch.isfinite(diff) & bits
            assert t.nonfinite == int((bits & ~torch.isfinite(diff)).sum())
            if fin.any():
                d = diff[fin]
                assert t.max_abs == pytest.approx(float(d.max()), rel=0, abs=0)
                rel = d / (vb[fin].abs() + 1e-12)
                assert t.max_rel == pytest.approx(float(rel.max()), rel=1e-6)
            # compare_ckpt: rms = ||A - B|| / sqrt(n), rel_rms = rms / (||B|| / sqrt(n) + 1e-12),
            # over the finite differences (identical elements contribute 0).
            n = va.numel()
            dd = torch.where(fin, diff, torch.zeros_like(diff)).double()
            rms = torch.linalg.norm(dd).item() / n ** 0.5
            vbf = torch.where(torch.isfinite(vb), vb, torch.zeros_like(vb)).double()
            rel_rms = rms / (torch.linalg.norm(vbf).item() / n ** 0.5 + 1e-12)
            assert t.rms == pytest.approx(rms, rel=1e-9, abs=1e-300)
            assert t.rel_rms == pytest.approx(rel_rms, rel=1e-9, abs=1e-300)
    assert len(report.mismatched()) > 0 and not report.bit_exact
    assert all("Value mismatch for" in line for line in report.lines())


def test_report_thresholds():
    t_ok = TensorDiff(100, 0, 0, 0.0, 1.0, 0.0, 0.0)
    t_small = TensorDiff(100, 3, 0, 1e-10, 1.0, 1e-5, 1e-4)
    t_nan = TensorDiff(100, 1, 1, 0.0, 1.0, 0.0, 0.0)
    r = VerifyReport({("w", "main"): t_ok, ("x", "main"): t_small, ("y", "param"): t_nan})
    assert r.elements == 300 and r.mismatches == 4 and not r.bit_exact
    assert r.mismatched() == [("x", "main"), ("y", "param")]
    assert r.mismatched(rel_rms_thresh=1e-3) == [("y", "param")]   # compare_ckpt's default threshold
    assert t_small.rel_rms == pytest.approx((1e-10 / 100) ** 0.5 / ((1.0 / 100) ** 0.5 + 1e-12))


def test_compare_abi_argument_checks():
    t = np.zeros(1, dtype=_native.SEGMENT_DTYPE)
    t[0] = (0, 0, 4, 0, 0, 0, 16, 1, 0, 0, 0, 0, 0, 0)
    plan = _native.Plan(t, [1024], [1024])
    with pytest.raises(_native.EmrsError) as e:
        plan.compare([0x1000], [0x2000], n_groups=0)
    assert e.value.code == -1
    with pytest.raises(_native.EmrsError) as e:
        plan.compare([0x1000], [0x2000], groups=np.array([3]), n_groups=3)
    assert e.value.code == -1
    with pytest.raises(ValueError):
        plan.compare([0x1000], [0x2000], groups=np.array([0, 1]), n_groups=3)
    if not torch.cuda.is_available():
        with pytest.raises(_native.EmrsError) as e:
            plan.compare([0x1000], [0x2000], groups=np.array([2]), n_groups=3)
        assert e.value.code == -6
