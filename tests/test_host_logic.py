"""Host-side logic of the package (no GPU): partial-attention plans, PositionMapping, module
aliases, the sequential-copy resolution of NoPE V moves, the position normalisation of
apply_rope_delta_inplace, the inv_freq table, and rejection of CPU tensors."""

from __future__ import annotations

import random
import sys

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from semblend_amd import compat
from semblend_amd import partial_attention as pa
from semblend_amd import rope_correction as rc
from semblend_amd import triton_kernels as tk
from semblend_amd.pipeline import PositionMapping

# ---- plans (synapse_kv_connector/tests/test_partial_attention.py) ----

COPY = "copy_from_donor"


def _acts(spec):
    out = []
    for kind, t, d in spec:
        a = {"action": kind, "targetPos": t}
        if d is not None:
            a["donorPos"] = d
        out.append(a)
    return out


def test_plan_basic():
    plan = pa.build_attention_plan(
        "d1", 5, 5, [0, 1, 3, 4], [2],
        _acts([(COPY, 0, 0), (COPY, 1, 1), ("placeholder", 2, None), (COPY, 3, 3), (COPY, 4, 4)]),
        num_layers=4)
    assert (plan.target_len, plan.donor_len, plan.donor_id) == (5, 5, "d1")
    assert (plan.num_reuse_positions, plan.num_partial_positions, plan.num_full_layers) == (4, 1, 0)
    assert len(plan.layer_masks) == 4
    assert abs(plan.computation_ratio - 0.2) < 1e-6
    np.testing.assert_array_equal(pa.compute_attention_mask(plan, 0),
                                  [False, False, True, False, False])
    assert pa.compute_attention_mask(plan, 0).dtype == bool
    assert pa.compute_donor_kv_indices(plan, 1) == [(0, 0), (1, 1), (3, 3), (4, 4)]


def test_plan_layer_hints_and_ratio():
    plan = pa.build_attention_plan(
        "d2", 4, 4, [0, 1, 2], [3],
        _acts([(COPY, 0, 0), (COPY, 1, 1), (COPY, 2, 2), ("placeholder", 3, None)]),
        layer_hints=[{"recomputeAll": False, "deviationScore": 0.1},
                     {"recomputeAll": True, "deviationScore": 0.5},
                     {"recompute_all": False, "deviation_score": 0.2},
                     {"recomputeAll": True, "deviationScore": 0.8}],
        num_layers=4)
    assert plan.num_full_layers == 2
    assert [m.recompute_all for m in plan.layer_masks] == [False, True, False, True]
    assert plan.layer_masks[2].deviation_score == 0.2
    assert abs(plan.computation_ratio - 0.625) < 1e-6
    assert pa.compute_attention_mask(plan, 1).all()
    assert pa.compute_donor_kv_indices(plan, 1) == []
    assert pa.compute_attention_mask(plan, 99).all()
    assert pa.compute_donor_kv_indices(plan, 99) == []


def test_plan_full_recompute_and_full_reuse():
    plan = pa.build_attention_plan("d3", 3, 3, [], [0, 1, 2],
                                   _acts([("placeholder", i, None) for i in range(3)]), num_layers=2)
    assert plan.num_partial_positions == 3 and abs(plan.computation_ratio - 1.0) < 1e-6
    plan = pa.build_attention_plan("d4", 3, 3, [0, 1, 2], [],
                                   _acts([(COPY, i, i) for i in range(3)]), num_layers=2)
    assert plan.num_reuse_positions == 3 and abs(plan.computation_ratio) < 1e-6


def test_plan_ignores_recompute_action():
    """build_attention_plan maps only copy_from_donor and placeholder
    (semblend_core/partial_attention.py:140-156): a "recompute" slot adds no mask entry."""
    plan = pa.build_attention_plan("d", 3, 3, [0], [1, 2],
                                   _acts([(COPY, 0, 0), ("recompute", 1, None),
                                          ("placeholder", 2, None)]), num_layers=1)
    np.testing.assert_array_equal(pa.compute_attention_mask(plan, 0), [False, False, True])
    assert plan.num_partial_positions == 2


def test_multi_donor_plan():
    acts = [{"action": COPY, "targetPos": 0, "donorPos": 4, "donorId": "a"},
            {"action": COPY, "targetPos": 1, "donorPos": 9, "donorId": "b"},
            {"action": COPY, "targetPos": 2, "donorPos": 5, "donorId": "a"},
            {"action": "recompute", "targetPos": 3},
            {"action": "placeholder", "targetPos": 4}]
    plan = pa.build_multi_donor_attention_plan(5, acts, num_layers=3)
    assert plan.donor_id == "a" and plan.donor_len == 10
    assert plan.donor_map == ((0, "a"), (1, "b"), (2, "a"))
    assert (plan.num_reuse_positions, plan.num_partial_positions) == (3, 1)
    np.testing.assert_array_equal(pa.compute_attention_mask(plan, 0),
                                  [False, False, False, True, False])
    assert pa.compute_donor_kv_indices(plan, 2) == [(4, 0), (9, 1), (5, 2)]
    assert abs(plan.computation_ratio - 1 / 5) < 1e-9
    empty = pa.build_multi_donor_attention_plan(0, [], num_layers=0)
    assert empty.donor_id == "" and empty.computation_ratio == 1.0


def test_multi_donor_position_mapping():
    # the reference suite's cases (tests/core/test_multi_donor_types.py:69-123), restated
    from semblend_amd.multi_donor import MultiDonorPositionMapping as M
    m = M(donor_ids=("d1", "d2"), donor_positions=(0, 256), target_positions=(0, 256))
    with pytest.raises(AttributeError):
        m.donor_ids = ()  # type: ignore[misc]
    assert M(("d1", "d1", "d2"), (0, 1, 100), (0, 1, 200)).num_pairs == 3
    assert not M(("d1",), (5,), (5,)).needs_correction
    assert M(("d1",), (5,), (10,)).needs_correction
    d1 = M(("d1", "d2", "d1", "d2"), (0, 100, 1, 101), (0, 200, 1, 201)).for_donor("d1")
    assert (d1.num_pairs, d1.donor_ids, d1.donor_positions, d1.target_positions) == \
        (2, ("d1", "d1"), (0, 1), (0, 1))
    assert M().num_pairs == 0 and not M().needs_correction


def test_composite_pairs():
    from semblend_amd.multi_donor import MultiDonorPositionMapping as M, composite_pairs
    m = M(("b", "a", "b", "c"), (7, 3, 8, 0), (10, 11, 12, 13))
    order, didx, dpos, tpos = composite_pairs(m)
    assert order == ("b", "a", "c")
    np.testing.assert_array_equal(didx, [0, 1, 0, 2])
    np.testing.assert_array_equal(dpos, [7, 3, 8, 0])
    np.testing.assert_array_equal(tpos, [10, 11, 12, 13])
    assert didx.dtype == np.int32 and dpos.dtype == np.int32 and tpos.dtype == np.int32
    order, didx, _, _ = composite_pairs(m, ("c", "b", "a"))
    np.testing.assert_array_equal(didx, [1, 2, 1, 0])
    with pytest.raises(ValueError, match="not in donor_order"):
        composite_pairs(m, ("a", "b"))
    with pytest.raises(ValueError, match="distinct"):
        composite_pairs(M(("a", "b"), (0, 1), (5, 5)))
    with pytest.raises(ValueError, match="length"):
        composite_pairs(M(("a",), (0, 1), (5, 6)))


def test_composite_pairs_from_plan():
    from semblend_amd.multi_donor import composite_pairs_from_plan
    acts = [{"action": COPY, "targetPos": 0, "donorPos": 4, "donorId": "a"},
            {"action": COPY, "targetPos": 1, "donorPos": 9, "donorId": "b"},
            {"action": COPY, "targetPos": 2, "donorPos": 5},
            {"action": "recompute", "targetPos": 3}]
    plan = pa.build_multi_donor_attention_plan(4, acts, num_layers=2)
    m = composite_pairs_from_plan(plan, 1)
    # position 2 has no donorId: it belongs to the plan's primary donor ("a": tie -> first)
    assert m.donor_ids == ("a", "b", plan.donor_id)
    assert m.donor_positions == (4, 9, 5) and m.target_positions == (0, 1, 2)
    full = pa.build_multi_donor_attention_plan(
        4, acts, layer_hints=[{"recomputeAll": True}], num_layers=2)
    assert composite_pairs_from_plan(full, 0).num_pairs == 0


def test_group_pairs_by_chunk():
    from semblend_amd.loader import group_pairs_by_chunk
    d = [700, 5, 256, 300, -1, 1024, 10, 511, 512]
    t = [0, 1, 2, 3, 4, 5, 6, 7, 8]
    arr, off = group_pairs_by_chunk(d, t, 256, 3)
    # chunk 0: d 5, 10 (pair order kept); chunk 1: 256, 300, 511; chunk 2: 700, 512;
    # d = -1 and d = 1024 (chunk 4 of 3) dropped
    np.testing.assert_array_equal(arr[0], [5, 10, 256, 300, 511, 700, 512])
    np.testing.assert_array_equal(arr[1], [1, 6, 2, 3, 7, 0, 8])
    np.testing.assert_array_equal(arr[2], 0)
    np.testing.assert_array_equal(off, [0, 2, 5, 7])
    assert arr.dtype == np.int32
    # brute force on random input: every kept pair in its chunk's run, runs in pair order
    rng = np.random.default_rng(3)
    d = rng.integers(-50, 3000, 500)
    t = rng.permutation(500)
    arr, off = group_pairs_by_chunk(d, t, 128, 20)
    kept = [(int(a), int(b)) for a, b in zip(d, t) if 0 <= a < 128 * 20]
    for c in range(20):
        want = [p for p in kept if p[0] // 128 == c]
        got = list(zip(arr[0, off[c]:off[c + 1]].tolist(), arr[1, off[c]:off[c + 1]].tolist()))
        assert got == want
    with pytest.raises(ValueError):
        group_pairs_by_chunk([1, 2], [3], 256, 1)


def test_plan_types_frozen_and_enum_values():
    m = pa.PositionMask(target_pos=0, mode=pa.AttentionMode.REUSE, donor_pos=3)
    assert m.donor_pos == 3
    assert pa.PositionMask(1, pa.AttentionMode.PARTIAL).donor_pos is None
    with pytest.raises(AttributeError):
        m.target_pos = 1  # type: ignore[misc]
    assert [e.value for e in pa.AttentionMode] == ["full", "reuse", "partial", "skip_layer"]
    assert pa.LayerMask(0, False, 0.0).verification_source == "bathtub"


def test_position_mapping():
    assert not PositionMapping([0, 1, 2], [0, 1, 2]).needs_correction
    pm = PositionMapping([0, 1, 2, 3], [2, 3, 0, 1])
    assert pm.needs_correction and pm.num_pairs == 4
    assert PositionMapping().num_pairs == 0


def test_compat_aliases():
    names = compat.install()
    assert "semblend_core.rope_correction" in names
    import semblend_core.rope_correction as a  # noqa: E402
    import synapse_kv_connector.triton_kernels as b  # noqa: E402
    from synapse_kv_connector.partial_attention import build_attention_plan  # noqa: E402
    assert a is rc and b is tk and build_attention_plan is pa.build_attention_plan
    assert a.HAS_TRITON is False
    for mod in ("semblend_core", "synapse_kv_connector"):
        sys.modules.pop(mod + ".rope_correction", None)


# ---- sequential V moves of nope_permute_paged_kv ----

def test_sequential_v_moves_matches_brute_force():
    rng = random.Random(7)
    for _ in range(200):
        n = rng.randint(1, 12)
        perm = [(rng.randrange(10), rng.randrange(10)) for _ in range(n)]
        state = {i: i for i in range(10)}   # position -> original row it holds
        for s, t in perm:
            state[t] = state[s]
        moves = rc._sequential_v_moves(perm)
        resolved = {i: i for i in range(10)}
        for t, s in moves:
            resolved[t] = s
        assert resolved == state, perm


# ---- apply_rope_delta_inplace host normalisation ----

def test_rotation_counts():
    counts, n = rc._rotation_counts([0, 5, 17, 17, 40, 127, 128, 300, -1, 64], 16, 8)
    assert n == 8  # 128 and 300 lie past the 8-block table
    assert counts == {0: 1, 5: 1, 17: 2, 40: 1, 127: 2, 64: 1}
    with pytest.raises(IndexError):
        rc._rotation_counts([-200], 16, 8)


def test_rotation_counts_agree_with_oracle_count():
    kv = torch.randn(10, 2, 2, 16, 8)
    bt = torch.tensor([4, 2, 0, 9], dtype=torch.int32)
    pos = [0, 3, 16, 16, 63, 64, 70, -1, -20]
    _, n = rc._rotation_counts(pos, 16, 4)
    assert n == ref_cpu.apply_rope_delta_inplace(kv, bt, pos, 3)


def test_delta_rounds_resolve_like_one_position_calls():
    """apply_rope_deltas_inplace_layers' host resolution: every (position, delta) entry is
    treated like a one-position apply_rope_delta_inplace call (the oracle's count per entry
    decides whether it is processed), each logical position's entries keep their list order
    across rounds, and no round holds a position twice."""
    rng = random.Random(7)
    bs, nbs = 16, 8
    pos = [rng.randrange(-nbs * bs, nbs * bs + 40) for _ in range(400)] + [5, 5, 5, -11, 117]
    dl = [rng.choice([0, rng.randrange(-3000, 3000)]) for _ in range(400)] + [1, 2, 3, 4, 5]
    rounds, n = rc._delta_rounds(pos, dl, bs, nbs)
    kv = torch.zeros(nbs, 2, 1, bs, 2)
    bt = torch.arange(nbs, dtype=torch.int32)
    want = []  # (logical position, delta) of the processed entries, in list order
    for p, d in zip(pos, dl):
        if ref_cpu.apply_rope_delta_inplace(kv, bt, [p], d):
            blk = p // bs
            want.append(((blk % nbs) * bs + p % bs, d))
    assert n == len(want)
    seen: dict[int, list[int]] = {}
    for rp, rd in rounds:
        assert rp.dtype == np.int32 and rd.dtype == np.int32
        assert len(set(rp.tolist())) == rp.size
        for p, d in zip(rp.tolist(), rd.tolist()):
            seen.setdefault(p, []).append(d)
    expect: dict[int, list[int]] = {}
    for p, d in want:
        expect.setdefault(p, []).append(d)
    assert seen == expect
    # -11 lies in the table's last block (-1), offset 5: logical 117, listed next with 5
    assert seen[5][-3:] == [1, 2, 3] and seen[117][-2:] == [4, 5]
    with pytest.raises(IndexError):
        rc._delta_rounds([-nbs * bs - 1], [3], bs, nbs)
    with pytest.raises(ValueError, match="2\\^31"):
        rc._delta_rounds([0], [1 << 31], bs, nbs)
    with pytest.raises(ValueError, match="length"):
        rc._delta_rounds([0, 1], [3], bs, nbs)
    assert rc._delta_rounds([0, 200], [0, 5], bs, nbs) == ([], 0)


def test_inv_freq_table_is_the_reference_expression():
    for base, d in ((10000.0, 128), (1e6, 128), (5e5, 64), (500.0, 32)):
        got = rc.inv_freq_table(base, d, torch.device("cpu"))
        assert torch.equal(got, ref_cpu.inv_freq(base, d))


# ---- no CPU path ----

def test_cpu_tensors_are_rejected():
    kv = torch.zeros(4, 2, 1, 4, 8)
    donor = torch.zeros(2, 1, 8, 8)
    idx = torch.tensor([0], dtype=torch.int32)
    bt = torch.tensor([0, 1], dtype=torch.int32)
    calls = [
        lambda: tk.scatter_donor_kv(torch.zeros(1, 2, 1, 8, 8), torch.zeros(1, 2, 1, 8, 8), idx, idx),
        lambda: tk.scatter_donor_kv_paged(kv, donor, bt, idx, idx),
        lambda: tk.partial_prefill_attention(torch.zeros(1, 4, 8), torch.zeros(1, 4, 8),
                                             torch.zeros(1, 4, 8), torch.ones(4, dtype=torch.bool)),
        lambda: tk.partial_prefill_attention_paged(torch.zeros(1, 1, 8), kv, bt, idx),
        lambda: rc.rope_correct_scatter_paged(kv, donor, bt, idx, idx),
        lambda: rc.rope_correct_k(torch.zeros(1, 4, 8), idx, idx, head_dim=8),
        lambda: rc.apply_rope_delta_inplace(kv, bt, [0], 3),
        lambda: rc.permute_paged_kv_with_rope(kv, bt, [(0, 1)]),
        lambda: rc.nope_permute_paged_kv(kv, bt, [(0, 1)]),
    ]
    for call in calls:
        with pytest.raises(RuntimeError, match="device tensors"):
            call()


def test_prepare_scatter_paged_layers_host_checks():
    """Checks made before any device work: layer counts, pair counts, and no launch for an
    empty pair set; CPU caches are refused (no CPU fallback)."""
    kv = [torch.zeros((4, 2, 2, 16, 64), dtype=torch.bfloat16) for _ in range(2)]
    donors = [torch.zeros((2, 2, 32, 64), dtype=torch.bfloat16) for _ in range(2)]
    bt = torch.arange(4, dtype=torch.int32)
    d = torch.arange(5, dtype=torch.int32)
    with pytest.raises(ValueError, match="same length"):
        rc.prepare_scatter_paged_layers(kv, donors[:1], bt, d, d)
    with pytest.raises(ValueError, match="differ in length"):
        rc.prepare_scatter_paged_layers(kv, donors, bt, d, d[:3])
    empty = torch.zeros(0, dtype=torch.int32)
    assert rc.prepare_scatter_paged_layers(kv, donors, bt, empty, empty) is None
    assert rc.rope_correct_scatter_paged_layers(kv, donors, bt, empty, empty) is kv
    with pytest.raises((ValueError, RuntimeError)):
        rc.prepare_scatter_paged_layers(kv, donors, bt, d, d)


def test_rows_repeat():
    """The load-policy hint of the multi-layer scatters: a donor row used by two pairs, per
    donor when donor indices are given; host sequences, numpy and CPU tensors alike."""
    from semblend_amd import _lib
    assert not _lib.rows_repeat([3, 1, 2])
    assert _lib.rows_repeat([3, 1, 3])
    assert not _lib.rows_repeat([])
    assert not _lib.rows_repeat(np.array([7]))
    assert _lib.rows_repeat(np.array([0, 5, 9, 5], dtype=np.int32))
    assert _lib.rows_repeat(torch.tensor([2, 2], dtype=torch.int32))
    # the same position of two donors is two rows; of one donor, one row
    assert not _lib.rows_repeat([4, 4], donor_index=[0, 1])
    assert _lib.rows_repeat([4, 4, 4], donor_index=[0, 1, 1])
    # negative positions (skipped pairs) and large positions keep distinct keys
    assert not _lib.rows_repeat([-1, 2**31 - 1], donor_index=[1, 0])
    assert _lib.scatter_flags(True) == _lib.SB_SCATTER_REPEATED_DONOR_ROWS == 1
    assert _lib.scatter_flags(False) == 0


def test_pair_length_mismatch_is_rejected_before_launch():
    """A target list shorter than the donor list would make the kernels read past it: every
    scatter entry refuses it with ValueError before looking at the device (CPU tensors here,
    so reaching the device check would raise RuntimeError instead)."""
    kv = torch.zeros(4, 2, 1, 4, 8)
    donor = torch.zeros(2, 1, 8, 8)
    bt = torch.tensor([0, 1], dtype=torch.int32)
    d = torch.tensor([0, 1, 2], dtype=torch.int32)
    t = torch.tensor([0, 1], dtype=torch.int32)
    flat = torch.zeros(1, 2, 1, 8, 8)
    calls = [
        lambda: tk.scatter_donor_kv(flat, flat.clone(), d, t),
        lambda: tk.scatter_donor_kv_paged(kv, donor, bt, d, t),
        lambda: tk.scatter_donor_kv_paged_layers([kv], [donor], bt, d, t),
        lambda: rc.rope_correct_scatter_paged(kv, donor, bt, d, t),
        lambda: rc.rope_correct_scatter_paged_layers([kv], [donor], bt, d, t),
    ]
    for call in calls:
        with pytest.raises(ValueError, match="differ in length"):
            call()


def test_layout_detection_and_empty():
    """Engine cache layouts resolve to the standard [NB, 2, H, bs, D] view; unknown layout
    names are refused; an empty permutation prepares nothing."""
    vllm = torch.zeros(2, 12, 16, 4, 64)
    assert rc.paged_layout(vllm)[:4] == (12, 4, 16, 64)
    assert rc.standard_view(vllm).shape == (12, 2, 4, 16, 64)
    std = torch.zeros(12, 2, 4, 16, 64)
    assert rc.paged_layout(std)[:4] == (12, 4, 16, 64)
    with pytest.raises(ValueError):
        rc.paged_layout(std, "nhd")
    assert rc.prepare_permute_paged_kv_layers([std], torch.zeros(2), []) is None


def test_group_pairs_by_donor():
    """Grouping for the donor-grouped composite launch: unknown donors dropped, pairs in donor
    order (stable within a donor), each donor's run padded with (-1, -1) to a multiple of the
    alignment except the last of its launch, launches of at most 16 donors."""
    from semblend_amd.multi_donor import group_pairs_by_donor

    rng = np.random.default_rng(3)
    n, nd = 900, 20
    didx = rng.integers(-2, nd + 2, n)
    dpos = rng.integers(0, 5000, n)
    tpos = rng.permutation(20000)[:n]
    launches = group_pairs_by_donor(didx, dpos, tpos, nd, align=256)
    assert [(f, c) for f, c, *_ in launches] == [(0, 16), (16, 4)]
    seen = []
    for first, count, dp, tp, ends in launches:
        assert dp.dtype == np.int32 and tp.dtype == np.int32 and ends.dtype == np.int64
        assert ends[-1] == dp.size == tp.size
        assert all(e % 256 == 0 for e in ends[:-1]) and all(np.diff(ends) >= 0)
        start = 0
        for k, e in zip(range(first, first + count), ends):
            seg_d, seg_t = dp[start:e], tp[start:e]
            real = seg_t >= 0
            want = [(int(a), int(b)) for a, b, c in zip(dpos, tpos, didx) if c == k]
            assert list(zip(seg_d[real].tolist(), seg_t[real].tolist())) == want
            assert np.all(seg_d[~real] == -1) and not np.any(real[real.argmin():]) or real.all()
            seen += want
            start = e
    assert len(seen) == int(((didx >= 0) & (didx < nd)).sum())
    assert group_pairs_by_donor([5], [1], [2], 3) == []
