"""Checks that pin the oracle, written against an implementation namespace ``impl`` that
provides the oracle's function names (see oracle/ref_cpu.py).

Three kinds of check:
  * the reference's own test cases, restated (synapse_kv_connector/tests/
    test_triton_kernels.py, test_rope_correction.py) with the reference's tolerances;
  * float64 golden vectors written independently by tests/golden/make_golden.py;
  * invariants fixed by the mathematics (rotation group law, norm preservation, identity at
    delta 0, V untouched by RoPE, zero rows outside the compute mask).

tests/test_oracle_pinning.py runs every check against the oracle; tests/test_oracle_mutations.py
plants plausible mistakes in copies of the oracle and requires that some check fails.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"


def _gen(seed):
    return torch.Generator("cpu").manual_seed(seed)


def _randn(shape, seed, dtype=torch.float32):
    return torch.randn(shape, generator=_gen(seed)).to(dtype)


def apply_rope_from_scratch(x, positions, head_dim, rope_base=10000.0):
    """The reference suite's test oracle (test_rope_correction.py:14-31), restated:
    rotate row i of x (second-to-last dim) by positions[i], interleaved, in fp32."""
    inv = 1.0 / (rope_base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    result = x.clone().float()
    for i, pos in enumerate(positions):
        theta = float(pos) * inv
        c, s = torch.cos(theta), torch.sin(theta)
        even = result[..., i, 0::2].clone()
        odd = result[..., i, 1::2].clone()
        result[..., i, 0::2] = even * c - odd * s
        result[..., i, 1::2] = even * s + odd * c
    return result.to(x.dtype)


def _close(a, b, atol, rtol, msg=""):
    torch.testing.assert_close(a, b, atol=atol, rtol=rtol, msg=msg or None)


# ------------------------------------------------------------------------------------------
# RoPE: reference cases (test_rope_correction.py)
# ------------------------------------------------------------------------------------------

def check_rope_reference_cases(impl) -> None:
    # identity, :37-47
    k = _randn((4, 8, 128), 1, torch.float16)
    pos = torch.tensor([0, 3, 7], dtype=torch.int32)
    _close(impl.rope_correct_k(k, pos, pos, head_dim=128), k, 1e-3, 1e-3)
    # exact move 5 -> 10, :49-83
    raw = _randn((4, 1, 128), 2)
    k5 = apply_rope_from_scratch(raw, torch.tensor([5]), 128)
    k10 = apply_rope_from_scratch(raw, torch.tensor([10]), 128)
    padded = torch.zeros(4, 11, 128)
    padded[:, 5] = k5[:, 0]
    out = impl.rope_correct_k(padded, torch.tensor([5], dtype=torch.int32),
                              torch.tensor([10], dtype=torch.int32), head_dim=128)
    _close(out[:, 5], k10[:, 0], 1e-4, 1e-4)
    # reorder, :85-117
    raw = _randn((4, 4, 64), 3)
    dpos = torch.arange(4, dtype=torch.int32)
    tpos = torch.tensor([2, 3, 0, 1], dtype=torch.int32)
    out = impl.rope_correct_k(apply_rope_from_scratch(raw, dpos, 64), dpos, tpos, head_dim=64)
    _close(out, apply_rope_from_scratch(raw, tpos, 64), 1e-3, 1e-3)
    # negative delta, :119-144
    raw = _randn((2, 1, 64), 4)
    padded = torch.zeros(2, 101, 64)
    padded[:, 100] = apply_rope_from_scratch(raw, torch.tensor([100]), 64)[:, 0]
    out = impl.rope_correct_k(padded, torch.tensor([100], dtype=torch.int32),
                              torch.tensor([50], dtype=torch.int32), head_dim=64)
    _close(out[:, 100], apply_rope_from_scratch(raw, torch.tensor([50]), 64)[:, 0], 1e-3, 1e-3)
    # composition identity, :294-323
    k = _randn((2, 10, 64), 5)
    s1 = impl.rope_correct_k(k, torch.tensor([3], dtype=torch.int32),
                             torch.tensor([8], dtype=torch.int32), head_dim=64)
    s2 = impl.rope_correct_k(s1, torch.tensor([3], dtype=torch.int32),
                             torch.tensor([-2], dtype=torch.int32), head_dim=64)
    _close(s2[:, 3], k[:, 3], 1e-3, 1e-3)
    # bases, :325-353
    for base in (500.0, 10000.0, 1e6):
        raw = _randn((2, 1, 32), 6)
        padded = torch.zeros(2, 11, 32)
        padded[:, 0] = apply_rope_from_scratch(raw, torch.tensor([0]), 32, base)[:, 0]
        out = impl.rope_correct_k(padded, torch.tensor([0], dtype=torch.int32),
                                  torch.tensor([10], dtype=torch.int32), head_dim=32,
                                  rope_base=base)
        _close(out[:, 0], apply_rope_from_scratch(raw, torch.tensor([10]), 32, base)[:, 0],
               1e-3, 1e-3, f"base {base}")


def check_rope_paged_reference_cases(impl) -> None:
    nb, h, bs, d = 4, 2, 16, 64
    # V unchanged, :162-191
    kv = torch.zeros(nb, 2, h, bs, d)
    donor = _randn((2, h, 32, d), 7)
    bt = torch.arange(nb, dtype=torch.int32)
    dp = torch.tensor([0, 1, 2], dtype=torch.int32)
    tp = torch.tensor([5, 10, 15], dtype=torch.int32)
    impl.rope_correct_scatter_paged(kv, donor, bt, dp, tp)
    for a, b in zip(dp.tolist(), tp.tolist()):
        _close(kv[b // bs, 1, :, b % bs], donor[1, :, a], 1e-6, 1e-6)
    # K corrected, :193-233
    kv = torch.zeros(nb, 2, h, bs, d)
    raw = _randn((h, 1, d), 8)
    donor = torch.zeros(2, h, 32, d)
    donor[0, :, 3] = apply_rope_from_scratch(raw, torch.tensor([3]), d)[:, 0]
    donor[1] = _randn((h, 32, d), 9)
    impl.rope_correct_scatter_paged(kv, donor, bt, torch.tensor([3], dtype=torch.int32),
                                    torch.tensor([7], dtype=torch.int32))
    _close(kv[0, 0, :, 7], apply_rope_from_scratch(raw, torch.tensor([7]), d)[:, 0], 1e-3, 1e-3)
    # permute swap, :235-264
    kv = _randn((2, 2, h, bs, d), 10)
    v0, v1 = kv[0, 1, :, 0].clone(), kv[0, 1, :, 1].clone()
    impl.permute_paged_kv_with_rope(kv, torch.arange(2, dtype=torch.int32), [(0, 1), (1, 0)])
    _close(kv[0, 1, :, 1], v0, 1e-6, 1e-6)
    _close(kv[0, 1, :, 0], v1, 1e-6, 1e-6)


def check_nope_reference_cases(impl) -> None:
    """test_rope_correction.py:452-637: NoPE identity, NoPE == delta for many deltas, NoPE
    matches fresh RoPE at the target, V copied exactly."""
    def single(raw, pos, d, base=10000.0):
        return apply_rope_from_scratch(raw.unsqueeze(1), torch.tensor([pos]), d, base)[:, 0]

    def cache(h, d, seq, bs=16):
        nb = (seq + bs - 1) // bs + 2
        return (torch.zeros(nb, 2, h, bs, d, dtype=torch.float16),
                torch.arange((seq + bs - 1) // bs, dtype=torch.int32))

    raw = _randn((4, 64), 11)
    kv, bt = cache(4, 64, 32)
    kv[0, 0, :, 5] = single(raw, 5, 64).half()
    impl.nope_permute_paged_kv(kv, bt, [(5, 5)])
    _close(kv[0, 0, :, 5].float(), single(raw, 5, 64), 5e-3, 5e-3)
    raw = _randn((4, 128), 12)
    kv, bt = cache(4, 128, 64)
    kv[0, 0, :, 7] = single(raw, 7, 128).half()
    impl.nope_permute_paged_kv(kv, bt, [(7, 23)])
    _close(kv[1, 0, :, 7].float(), single(raw, 23, 128), 1e-2, 1e-2)
    for delta in (0, 1, 5, 50, 100, 256, 1000):
        raw = _randn((8, 128), 13)
        tgt = 5 + delta
        kd, bt = cache(8, 128, max(tgt + 16, 128))
        kn, _ = cache(8, 128, max(tgt + 16, 128))
        kd[0, 0, :, 5] = single(raw, 5, 128).half()
        kn[0, 0, :, 5] = single(raw, 5, 128).half()
        impl.permute_paged_kv_with_rope(kd, bt, [(5, tgt)])
        impl.nope_permute_paged_kv(kn, bt, [(5, tgt)])
        _close(kn[tgt // 16, 0, :, tgt % 16].float(), kd[tgt // 16, 0, :, tgt % 16].float(),
               5e-3, 5e-3, f"delta {delta}")
    kv, bt = cache(4, 64, 32)
    v = _randn((4, 64), 14, torch.float16)
    kv[0, 1, :, 2] = v
    impl.nope_permute_paged_kv(kv, bt, [(2, 10)])
    assert torch.equal(kv[0, 1, :, 10], v)


def check_nope_sequential_v(impl) -> None:
    """V rows move pair by pair in list order (rope_correction.py:650-653): after the swap
    [(0, 1), (1, 0)] both rows hold the original row 0."""
    kv = _randn((2, 2, 2, 16, 32), 15)
    v0 = kv[0, 1, :, 0].clone()
    impl.nope_permute_paged_kv(kv, torch.arange(2, dtype=torch.int32), [(0, 1), (1, 0)])
    assert torch.equal(kv[0, 1, :, 0], v0) and torch.equal(kv[0, 1, :, 1], v0)


def check_apply_rope_delta(impl) -> None:
    """apply_rope_delta_inplace: delta then -delta restores K (semblend_connector.py:609-616),
    V untouched, both layouts, the returned count, the delta-0 and empty shortcuts."""
    kv = _randn((6, 2, 2, 16, 64), 16)
    bt = torch.tensor([3, 1, 4, 0], dtype=torch.int32)
    orig = kv.clone()
    pos = [0, 7, 16, 33, 63, 64, 100]          # 64 and 100 lie past the 4-block table
    assert impl.apply_rope_delta_inplace(kv, bt, pos, 77) == 5
    assert torch.equal(kv[:, 1], orig[:, 1])
    assert not torch.allclose(kv[3, 0, :, 0], orig[3, 0, :, 0])
    impl.apply_rope_delta_inplace(kv, bt, pos, -77)
    _close(kv, orig, 1e-5, 1e-5)
    assert impl.apply_rope_delta_inplace(kv, bt, pos, 0) == 0
    assert impl.apply_rope_delta_inplace(kv, bt, [], 5) == 0
    # vLLM layout [2, NB, bs, H, D] must rotate the same rows the same way
    std = _randn((6, 2, 2, 16, 64), 17)
    vllm = std.permute(1, 0, 3, 2, 4).contiguous()
    impl.apply_rope_delta_inplace(std, bt, [5, 40], 9)
    impl.apply_rope_delta_inplace(vllm, bt, [5, 40], 9)
    assert torch.equal(vllm.permute(1, 0, 3, 2, 4), std)


# ------------------------------------------------------------------------------------------
# RoPE: float64 golden vectors and invariants
# ------------------------------------------------------------------------------------------

def check_rope_golden(impl) -> None:
    g = np.load(GOLDEN / "rope_golden.npz")
    i = 0
    while f"c{i}_raw" in g:
        base = float(g[f"c{i}_base"])
        k_at_d = torch.from_numpy(g[f"c{i}_k_at_d"])
        dpos = torch.from_numpy(g[f"c{i}_dpos"])
        tpos = torch.from_numpy(g[f"c{i}_tpos"])
        d = k_at_d.shape[-1]
        # place each cached row at its donor slot of a [H, S, D] tensor, one row per pair
        n = dpos.shape[0]
        local = torch.arange(n, dtype=torch.int32)
        out = impl.rope_correct_k(k_at_d, local, local + (tpos - dpos), head_dim=d,
                                  rope_base=base)
        want = torch.from_numpy(g[f"c{i}_corrected"])
        err = (out.double() - want).abs().max().item()
        assert err < 2e-5, f"case {i}: max error {err} vs the float64 correction"
        err_t = (out.double() - torch.from_numpy(g[f"c{i}_k_at_t"])).abs().max().item()
        assert err_t < 5e-5, f"case {i}: max error {err_t} vs RoPE computed at the target"
        i += 1
    assert i >= 4


def check_rope_invariants(impl) -> None:
    k = _randn((3, 40, 64), 18)
    pos = torch.arange(40, dtype=torch.int32)
    g = _gen(19)
    a = torch.randint(-500, 500, (40,), generator=g, dtype=torch.int32)
    b = torch.randint(-500, 500, (40,), generator=g, dtype=torch.int32)
    ra = impl.rope_correct_k(k, pos, pos + a, head_dim=64, rope_base=1e4)
    # norms of every interleaved pair are preserved
    def pn(x):
        return torch.sqrt(x[..., 0::2] ** 2 + x[..., 1::2] ** 2)
    _close(pn(ra), pn(k), 1e-5, 1e-5)
    # group law R(b) R(a) = R(a + b)
    rab = impl.rope_correct_k(ra, pos, pos + b, head_dim=64, rope_base=1e4)
    r_sum = impl.rope_correct_k(k, pos, pos + a + b, head_dim=64, rope_base=1e4)
    _close(rab, r_sum, 1e-4, 1e-4)
    # a rotation by +1 of pair i is by exactly inv_freq[i] radians: compare with cos/sin
    e = torch.zeros(1, 1, 64)
    e[..., 0::2] = 1.0
    r1 = impl.rope_correct_k(e, torch.tensor([0], dtype=torch.int32),
                             torch.tensor([1], dtype=torch.int32), head_dim=64, rope_base=1e4)
    f64 = 1.0 / 1e4 ** (np.arange(0, 64, 2) / 64.0)
    _close(r1[0, 0, 0::2].double(), torch.from_numpy(np.cos(f64)), 1e-6, 1e-6)
    _close(r1[0, 0, 1::2].double(), torch.from_numpy(np.sin(f64)), 1e-6, 1e-6)


# ------------------------------------------------------------------------------------------
# Scatter
# ------------------------------------------------------------------------------------------

def check_scatter_reference_cases(impl) -> None:
    # test_triton_kernels.py:82-168
    target = torch.zeros(2, 2, 4, 16, 32, dtype=torch.float16)
    donor = _randn((2, 2, 4, 8, 32), 20, torch.float16)
    dp = torch.tensor([0, 2, 4, 6], dtype=torch.int32)
    tp = torch.tensor([1, 3, 7, 12], dtype=torch.int32)
    impl.scatter_donor_kv(target, donor, dp, tp)
    for a, b in zip(dp.tolist(), tp.tolist()):
        assert torch.equal(target[:, :, :, b], donor[:, :, :, a])
    for p in (0, 2, 4):
        assert torch.all(target[:, :, :, p] == 0)
    full = torch.zeros(2, 2, 4, 16, 32, dtype=torch.float16)
    donor = _randn((2, 2, 4, 16, 32), 21, torch.float16)
    ar = torch.arange(16, dtype=torch.int32)
    impl.scatter_donor_kv(full, donor, ar, ar)
    assert torch.equal(full, donor)
    # test_triton_kernels.py:208-302
    kv = torch.zeros(8, 2, 2, 4, 16, dtype=torch.float16)
    donor = _randn((2, 2, 8, 16), 22, torch.float16)
    impl.scatter_donor_kv_paged(kv, donor, torch.tensor([3, 5], dtype=torch.int32),
                                torch.tensor([0, 4], dtype=torch.int32),
                                torch.tensor([1, 5], dtype=torch.int32))
    assert torch.equal(kv[3, :, :, 1], donor[:, :, 0])
    assert torch.equal(kv[5, :, :, 1], donor[:, :, 4])
    kv = torch.zeros(4, 2, 1, 4, 8, dtype=torch.float16)
    donor = _randn((2, 1, 4, 8), 23, torch.float16)
    impl.scatter_donor_kv_paged(kv, donor, torch.tensor([1], dtype=torch.int32),
                                torch.tensor([0, 1], dtype=torch.int32),
                                torch.tensor([2, 8], dtype=torch.int32))
    assert torch.equal(kv[1, :, :, 2], donor[:, :, 0])
    kv[1, :, :, 2] = 0
    assert torch.all(kv == 0)


def check_scatter_golden(impl) -> None:
    g = np.load(GOLDEN / "scatter_golden.npz")
    kv = torch.from_numpy(g["p_kv"].copy())
    impl.scatter_donor_kv_paged(kv, torch.from_numpy(g["p_donor"]), torch.from_numpy(g["p_bt"]),
                                torch.from_numpy(g["p_dpos"]), torch.from_numpy(g["p_tpos"]))
    assert torch.equal(kv.double(), torch.from_numpy(g["p_out"])), "paged scatter golden"
    tgt = torch.from_numpy(g["f_target"].copy())
    impl.scatter_donor_kv(tgt, torch.from_numpy(g["f_donor"]), torch.from_numpy(g["f_dpos"]),
                          torch.from_numpy(g["f_tpos"]))
    assert torch.equal(tgt.double(), torch.from_numpy(g["f_out"])), "flat scatter golden"


# ------------------------------------------------------------------------------------------
# Attention
# ------------------------------------------------------------------------------------------

def check_attention_reference_cases(impl) -> None:
    # test_triton_kernels.py:396-493
    q, k, v = (_randn((2, 8, 16), s) for s in (30, 31, 32))
    scale = 1.0 / math.sqrt(16)
    res = impl.partial_prefill_attention(q, k, v, torch.ones(8, dtype=torch.bool), scale)
    for h in range(2):
        for pos in range(8):
            w = torch.softmax(q[h, pos:pos + 1] @ k[h, :pos + 1].T * scale, dim=-1)
            _close(res[h, pos], (w @ v[h, :pos + 1]).squeeze(0), 1e-4, 1e-3)
    mask = torch.tensor([True, False] * 4)
    res = impl.partial_prefill_attention(q, k, v, mask)
    for pos in (1, 3, 5, 7):
        assert torch.all(res[:, pos] == 0)
    q1, k1, v1 = (_randn((1, 4, 8), s) for s in (33, 34, 35))
    res = impl.partial_prefill_attention(q1, k1, v1, torch.tensor([False, False, False, True]))
    w = torch.softmax(q1[0, 3:4] @ k1[0].T / math.sqrt(8), dim=-1)
    _close(res[0, 3], (w @ v1[0]).squeeze(0), 1e-4, 1e-3)
    res = impl.partial_prefill_attention(q1, k1, v1, torch.zeros(4, dtype=torch.bool))
    assert torch.all(res == 0)


def check_attention_golden(impl) -> None:
    g = np.load(GOLDEN / "attention_golden.npz")
    i = 0
    while f"d{i}_q" in g:
        out = impl.partial_prefill_attention(
            torch.from_numpy(g[f"d{i}_q"]), torch.from_numpy(g[f"d{i}_k"]),
            torch.from_numpy(g[f"d{i}_v"]), torch.from_numpy(g[f"d{i}_mask"]),
            float(g[f"d{i}_scale"]))
        err = (out.double() - torch.from_numpy(g[f"d{i}_out"])).abs().max().item()
        assert err < 1e-5, f"dense case {i}: max error {err}"
        i += 1
    out = impl.partial_attention_paged(torch.from_numpy(g["g_q"]), torch.from_numpy(g["g_kv"]),
                                       torch.from_numpy(g["g_bt"]), torch.from_numpy(g["g_pos"]))
    err = (out.double() - torch.from_numpy(g["g_out"])).abs().max().item()
    assert err < 1e-5, f"GQA paged case: max error {err}"


def check_gqa_matches_dense(impl) -> None:
    """Paged GQA attention equals the dense MHA computation on the gathered, head-expanded
    K/V (the reference computation applied per query head)."""
    nb, hkv, hq, bs, d, seq = 12, 2, 8, 16, 32, 150
    kv = _randn((nb, 2, hkv, bs, d), 40)
    bt = torch.randperm(nb, generator=_gen(41))[:10].to(torch.int32)
    pos = torch.tensor([0, 3, 17, 64, 99, 149], dtype=torch.int32)
    q = _randn((pos.shape[0], hq, d), 42)
    out = impl.partial_attention_paged(q, kv, bt, pos)
    t = torch.arange(seq)
    kd = kv[bt[t // bs].long(), 0, :, t % bs].permute(1, 0, 2)
    vd = kv[bt[t // bs].long(), 1, :, t % bs].permute(1, 0, 2)
    g = hq // hkv
    qd = torch.zeros(hq, seq, d)
    mask = torch.zeros(seq, dtype=torch.bool)
    for r, p in enumerate(pos.tolist()):
        qd[:, p] = q[r]
        mask[p] = True
    dense = impl.partial_prefill_attention(qd, kd.repeat_interleave(g, 0),
                                           vd.repeat_interleave(g, 0), mask)
    _close(out, dense[:, pos.long()].permute(1, 0, 2), 1e-5, 1e-5)


# ------------------------------------------------------------------------------------------
# Projection and orchestrator
# ------------------------------------------------------------------------------------------

def check_projection_and_prefill(impl) -> None:
    # test_triton_kernels.py:313-385
    x = _randn((8, 32), 50, torch.float16)
    w = _randn((48, 32), 51, torch.float16)
    b = _randn((48,), 52, torch.float16)
    out = impl.masked_qkv_projection(x, w, torch.ones(8, dtype=torch.bool), b)
    _close(out, torch.nn.functional.linear(x.float(), w.float(), b.float()).half(), 1e-2, 1e-2)
    mask = torch.tensor([True, False] * 4)
    out = impl.masked_qkv_projection(x, w, mask)
    assert torch.all(out[~mask] == 0) and not torch.any(torch.all(out[mask] == 0, dim=1))
    # test_triton_kernels.py:504-713
    seq, hid, h, d, L = 16, 32, 4, 8, 2
    hs = _randn((seq, hid), 53, torch.float16)
    donor = _randn((L, 2, h, 10, d), 54, torch.float16)
    wq = _randn((3 * h * d, hid), 55, torch.float16)
    wo = _randn((hid, h * d), 56, torch.float16)
    dp = torch.tensor([0, 2, 4, 6, 8], dtype=torch.int32)
    tp = torch.tensor([0, 3, 6, 9, 12], dtype=torch.int32)
    cm = torch.ones(seq, dtype=torch.bool)
    cm[tp.long()] = False
    out, kv, computed, reused, ratio = impl.partial_prefill(hs, donor, wq, wo, dp, tp, cm, h, d)
    assert (computed, reused) == (11, 5) and abs(ratio - 11 / 16) < 1e-9
    assert out.shape == (seq, hid) and kv.shape == (L, 2, h, seq, d)
    for a, c in zip(dp.tolist(), tp.tolist()):
        assert torch.equal(kv[:, :, :, c], donor[:, :, :, a])
    assert torch.all(out[~cm] == 0)


# ------------------------------------------------------------------------------------------
# Orchestrator values (partial_prefill, triton_kernels.py:809-923)
# ------------------------------------------------------------------------------------------

def _prefill_values_case(seed, dtype):
    """Eight positions: computed {0, 2, 5, 7}; reused {1, 3, 4} from donor positions
    {0, 2, 1}; position 6 is a reuse position that no pair covers (its K/V stay zero). Three
    layers of distinct donor rows; hidden size equal to heads x head_dim, so the output
    projection is square and a transposed one changes values rather than shapes."""
    seq, h, d, layers = 8, 2, 4, 3
    hid = h * d
    hs = (0.5 * _randn((seq, hid), seed)).to(dtype)
    donor = _randn((layers, 2, h, 5, d), seed + 1, dtype)
    wo = (0.5 * _randn((hid, h * d), seed + 2)).to(dtype)
    dp = torch.tensor([0, 2, 1], dtype=torch.int32)
    tp = torch.tensor([1, 3, 4], dtype=torch.int32)
    cm = torch.ones(seq, dtype=torch.bool)
    cm[torch.tensor([1, 3, 4, 6])] = False
    return hs, donor, wo, dp, tp, cm, h, d


def _prefill_float64(hs, donor, wqkv, wo, dp, tp, cm, h, d, bqkv=None, bo=None, scale=None):
    """The orchestrator's result computed independently in float64 with numpy, from what the
    reference's stages state (triton_kernels.py:786-799, 831-897): the projection of every
    computed position is rounded once to the input dtype; each computed row attends
    causally, per head, over keys whose K/V are the new projection at computed positions,
    layer 0's donor row at reused positions a pair covers, and zero elsewhere; heads are
    concatenated and multiplied by the output projection; reuse rows are zero. Returns the
    output (float64) and the expected new K and V of every computed position."""
    dtype = hs.dtype
    seq, hid = hs.shape
    f = h * d
    x = hs.double().numpy()
    w = wqkv.double().numpy()
    proj = x @ w.T
    if bqkv is not None:
        proj = proj + bqkv.double().numpy()[None, :]
    # rounded as an fp32 GEMM whose result is cast to the input dtype
    proj = torch.from_numpy(proj).float().to(dtype).double().numpy()
    comp = cm.numpy().astype(bool)
    donor64 = donor.double().numpy()
    src = {int(t): int(s) for s, t in zip(dp.tolist(), tp.tolist())}
    keys = np.zeros((seq, h, d))
    vals = np.zeros((seq, h, d))
    for p in range(seq):
        if comp[p]:
            keys[p] = proj[p, f:2 * f].reshape(h, d)
            vals[p] = proj[p, 2 * f:3 * f].reshape(h, d)
        elif p in src:
            keys[p] = donor64[0, 0, :, src[p], :]
            vals[p] = donor64[0, 1, :, src[p], :]
    sc = 1.0 / math.sqrt(d) if scale is None else scale
    wo64 = wo.double().numpy()
    out = np.zeros((seq, wo64.shape[0]))
    for i in range(seq):
        if not comp[i]:
            continue
        flat = np.zeros(f)
        for hh in range(h):
            qv = proj[i, hh * d:(hh + 1) * d]
            s = np.array([sc * float(np.dot(qv, keys[k, hh])) for k in range(i + 1)])
            p = np.exp(s - s.max())
            p /= p.sum()
            flat[hh * d:(hh + 1) * d] = sum(p[k] * vals[k, hh] for k in range(i + 1))
        out[i] = wo64 @ flat
        if bo is not None:
            out[i] += bo.double().numpy()
    return out, keys, vals


def check_partial_prefill_selector_closed_form(impl) -> None:
    """Selector weights make every stage identifiable and exact. Q weights are zero, so every
    computed row weights its keys 0..i equally; K features copy hidden element c, V features
    copy -2 x element (c + 1) mod hidden (exact in every dtype). Then:
      * the row at position 0 attends to itself only: out[0] = W_o . v_new[0] + b;
      * out[i] = W_o . mean(V over keys 0..i) + b, where V is the new projection at computed
        positions, layer 0's donor row at covered reuse positions, zero at position 6;
      * every layer's cache holds the new K (plane 0) and V (plane 1) at computed positions,
        the layer's own donor rows at covered reuse positions, zeros at position 6;
      * reuse rows of the output are zero."""
    for dtype in (torch.float32, torch.bfloat16):
        hs, donor, wo, dp, tp, cm, h, d = _prefill_values_case(300, dtype)
        seq, hid = hs.shape
        f = h * d
        w = torch.zeros((3 * f, hid))
        for c in range(f):
            w[f + c, c] = 1.0
            w[2 * f + c, (c + 1) % hid] = -2.0
        w = w.to(dtype)
        bo = (0.25 * _randn((hid,), 303)).to(dtype)
        out, kv, computed, reused, ratio = impl.partial_prefill(hs, donor, w, wo, dp, tp, cm,
                                                                h, d, output_bias=bo)
        assert (computed, reused) == (4, 4) and abs(ratio - 0.5) < 1e-12
        x = hs.double()
        k_new = x[:, :f].reshape(seq, h, d)
        v_new = -2.0 * torch.roll(x, -1, dims=1)[:, :f].reshape(seq, h, d)
        merged_v = torch.zeros((seq, h, d), dtype=torch.float64)
        for p in range(seq):
            if bool(cm[p]):
                merged_v[p] = v_new[p]
        for s, t in zip(dp.tolist(), tp.tolist()):
            merged_v[t] = donor[0, 1, :, s].double()
        wo64, bo64 = wo.double(), bo.double()
        # closed form of row 0, then of every computed row
        row0 = wo64 @ v_new[0].reshape(-1) + bo64
        want = torch.zeros((seq, hid), dtype=torch.float64)
        for i in torch.where(cm)[0].tolist():
            want[i] = wo64 @ merged_v[:i + 1].mean(dim=0).reshape(-1) + bo64
        assert torch.allclose(want[0], row0)
        eps = 2.0 ** -20 if dtype == torch.float32 else 2.0 ** -8
        bound = (wo64.abs() @ merged_v.abs().amax(dim=0).reshape(-1) + bo64.abs()) * eps
        err = (out.double() - want).abs()
        assert bool((err <= bound[None, :]).all()), f"{dtype}: output max error {err.max()}"
        assert torch.all(out[~cm] == 0)
        # the cache of every layer
        for layer in range(donor.shape[0]):
            for p in range(seq):
                if bool(cm[p]):
                    assert torch.equal(kv[layer, 0, :, p].double(), k_new[p])
                    assert torch.equal(kv[layer, 1, :, p].double(), v_new[p])
            for s, t in zip(dp.tolist(), tp.tolist()):
                assert torch.equal(kv[layer, :, :, t], donor[layer, :, :, s])
            assert not bool(kv[layer, :, :, 6].any())


def check_partial_prefill_float64(impl) -> None:
    """Random weights and biases (Q, K and V all live, non-default scale): the oracle's
    output within fp32 rounding (fp32) or one ulp plus carried projection rounding (bf16)
    of the float64 computation above, and the new K/V in every layer equal to the projection
    rounded once."""
    for dtype, seed in ((torch.float32, 310), (torch.bfloat16, 320)):
        hs, donor, wo, dp, tp, cm, h, d = _prefill_values_case(seed, dtype)
        seq, hid = hs.shape
        f = h * d
        wqkv = (0.5 * _randn((3 * f, hid), seed + 5)).to(dtype)
        bqkv = (0.25 * _randn((3 * f,), seed + 6)).to(dtype)
        bo = (0.25 * _randn((hid,), seed + 7)).to(dtype)
        out, kv, *_ = impl.partial_prefill(hs, donor, wqkv, wo, dp, tp, cm, h, d,
                                           qkv_bias=bqkv, output_bias=bo, scale=0.3)
        want, keys, vals = _prefill_float64(hs, donor, wqkv, wo, dp, tp, cm, h, d, bqkv, bo,
                                            scale=0.3)
        want = torch.from_numpy(want)
        scale_ref = wo.double().abs() @ torch.from_numpy(np.abs(vals).max(axis=0)).reshape(-1)
        if dtype == torch.float32:
            tol = 1e-5 * scale_ref[None, :] + 1e-6
        else:
            ulp = 2.0 ** (torch.floor(torch.log2(want.abs().clamp_min(2.0 ** -14))) - 7)
            tol = ulp + 2.0 ** -10 * scale_ref[None, :]
        err = (out.double() - want).abs()
        assert bool((err <= tol).all()), f"{dtype}: output max error {err.max()}"
        # new K/V: bf16 rows equal the rounded projection (these seeds hold no rounding
        # ties); fp32 rows within fp32 rounding of sum |x w| + |b|
        dot = hs.double().abs() @ wqkv.double().abs().T + bqkv.double().abs()
        for layer in range(donor.shape[0]):
            for p in torch.where(cm)[0].tolist():
                for plane, want_rows, lo in ((0, keys, f), (1, vals, 2 * f)):
                    got = kv[layer, plane, :, p].double()
                    exp = torch.from_numpy(want_rows[p])
                    if dtype == torch.float32:
                        bar = 2.0 ** -21 * dot[p, lo:lo + f].reshape(h, d)
                        assert bool(((got - exp).abs() <= bar).all())
                    else:
                        assert torch.equal(got, exp)



# ------------------------------------------------------------------------------------------
# Multi-donor (composite) scatter: concatenation identities
# ------------------------------------------------------------------------------------------

def _composite_case(dtype, lens, seed, n_pairs=40):
    """Donors of the given lengths, distinct targets over a permuted block table, pairs
    spread over the donors plus pairs that must be skipped (unknown donor ids, donor
    positions past their donor's end)."""
    bs, nb, h, d = 4, 16, 2, 16
    g = _gen(seed)
    donors = [_randn((2, h, n, d), seed + 1 + k, dtype) for k, n in enumerate(lens)]
    tpos = torch.randperm(nb * bs, generator=g)[:n_pairs]
    didx = torch.randint(0, len(lens), (n_pairs,), generator=g)
    dpos = torch.tensor([int(torch.randint(0, lens[k], (1,), generator=g)) for k in didx])
    bad = torch.randperm(nb * bs, generator=g)
    bad = bad[~torch.isin(bad, tpos)][:3]
    bad_idx = torch.tensor([len(lens), -1, 0])
    bad_pos = torch.tensor([0, 0, lens[0]])
    bt = torch.randperm(nb + 5, generator=g)[:nb].to(torch.int32)
    cache = _randn((nb + 5, 2, h, bs, d), seed + 20, dtype)
    return (donors, bt, cache, didx, dpos, tpos, torch.cat([didx, bad_idx]),
            torch.cat([dpos, bad_pos]), torch.cat([tpos, bad]))


def check_composite_concatenation(impl) -> None:
    """Plain copies: a composite scatter from donors A, B, C equals one single-donor scatter
    from cat(A, B, C) along the sequence, each pair's donor position shifted by its donor's
    offset in the concatenation (ragged donor lengths; skipped pairs left out)."""
    for dtype in (torch.float32, torch.bfloat16):
        lens = [64, 20, 12]
        donors, bt, cache, didx, dpos, tpos, cidx, cdpos, ctpos = _composite_case(dtype, lens, 50)
        offs = torch.tensor([0, 64, 84])
        want = impl.scatter_donor_kv_paged(cache.clone(), torch.cat(donors, dim=2), bt,
                                           dpos + offs[didx], tpos)
        got = impl.composite_scatter_paged(cache.clone(), donors, bt, cidx, cdpos, ctpos,
                                           rope=False)
        assert torch.equal(got, want)


def check_composite_rope_concatenation(impl) -> None:
    """RoPE: the same identity with targets shifted as well, so every delta t - d is kept;
    the block table is repeated once per donor and every donor but the last spans exactly
    one table (64 positions), so a shifted target names the same physical slot."""
    for dtype in (torch.float32, torch.bfloat16):
        lens = [64, 64, 12]
        donors, bt, cache, didx, dpos, tpos, cidx, cdpos, ctpos = _composite_case(dtype, lens, 60)
        offs = torch.tensor([0, 64, 128])
        want = impl.rope_correct_scatter_paged(cache.clone(), torch.cat(donors, dim=2),
                                               bt.repeat(3), dpos + offs[didx],
                                               tpos + offs[didx], rope_base=500.0)
        got = impl.composite_scatter_paged(cache.clone(), donors, bt, cidx, cdpos, ctpos,
                                           rope=True, rope_base=500.0)
        assert torch.equal(got, want)
        # and the rotation is not a copy: K differs from the plain composite somewhere
        plain = impl.composite_scatter_paged(cache.clone(), donors, bt, cidx, cdpos, ctpos,
                                             rope=False)
        assert torch.equal(got[:, 1], plain[:, 1]) and not torch.equal(got[:, 0], plain[:, 0])



# ------------------------------------------------------------------------------------------
# Compacted GQA projection with the K/V write (qkv_project_paged)
# ------------------------------------------------------------------------------------------

def _proj_case(seed, h, hkv, d, hidden, seq=40, nb=6, bs=8, dtype=torch.bfloat16):
    g = _gen(seed)
    x = _randn((seq, hidden), seed + 1, dtype)
    pos = torch.randperm(seq, generator=g)[:17].sort().values.to(torch.int32)
    bt = torch.randperm(nb + 2, generator=g)[:nb].to(torch.int32)
    cache = _randn((nb + 2, 2, hkv, bs, d), seed + 2, dtype)
    return x, pos, bt, cache


def check_qkv_projection_mha(impl) -> None:
    """MHA, no RoPE: the compacted projection equals the reference's masked projection on
    the computed rows (Q, and the K/V now in the cache), bias included."""
    h, d, hidden = 4, 8, 24
    x, pos, bt, cache = _proj_case(70, h, h, d, hidden)
    w = _randn((3 * h * d, hidden), 73, torch.bfloat16)
    b = _randn((3 * h * d,), 74, torch.bfloat16)
    mask = torch.zeros(x.shape[0], dtype=torch.bool)
    mask[pos.long()] = True
    dense = impl.masked_qkv_projection(x, w, mask, b)
    kv = cache.clone()
    q = impl.qkv_project_paged(x, w, pos, kv, bt, h, h, d, qkv_bias=b)
    assert torch.equal(q.reshape(len(pos), -1), dense[pos.long(), :h * d])
    for r, p in enumerate(pos.tolist()):
        pb, off = int(bt[p // 8]), p % 8
        assert torch.equal(kv[pb, 0, :, off].reshape(-1), dense[p, h * d:2 * h * d])
        assert torch.equal(kv[pb, 1, :, off].reshape(-1), dense[p, 2 * h * d:])


def check_qkv_projection_layout(impl) -> None:
    """GQA feature layout and row gather, closed form: with selector weights (Q rows pick
    -x[j], K rows x[j], V rows 2 x[j + 1]) every output is a copy of an input element, so
    Q [R, Hq, D], K and V [Hkv, D] per position are fixed exactly; slots past the block
    table are not written; a position past the hidden states gives a zero Q row."""
    h, hkv, d, hidden = 4, 2, 8, 40
    x, pos, bt, cache = _proj_case(80, h, hkv, d, hidden)
    qf, kf = h * d, hkv * d
    w = torch.zeros((qf + 2 * kf, hidden))
    for j in range(qf):
        w[j, j % hidden] = -1.0
    for j in range(kf):
        w[qf + j, j] = 1.0
        w[qf + kf + j, j + 1] = 2.0
    w = w.to(torch.bfloat16)
    pos = torch.cat([pos, torch.tensor([47, x.shape[0]], dtype=torch.int32)])  # 47: past table
    xx = torch.cat([x, _randn((8, hidden), 81, torch.bfloat16)])  # rows 40..47 exist
    kv = cache.clone()
    q = impl.qkv_project_paged(xx, w, pos, kv, bt, h, hkv, d)
    for r, p in enumerate(pos.tolist()):
        if p >= xx.shape[0]:
            assert torch.all(q[r] == 0)
            continue
        want_q = torch.stack([-xx[p, j % hidden] for j in range(qf)]).reshape(h, d)
        assert torch.equal(q[r], want_q)
        if p // 8 >= bt.shape[0]:
            continue
        pb, off = int(bt[p // 8]), p % 8
        assert torch.equal(kv[pb, 0, :, off], xx[p, :kf].reshape(hkv, d))
        assert torch.equal(kv[pb, 1, :, off], 2 * xx[p, 1:kf + 1].reshape(hkv, d))
    # untouched elsewhere: only slots of computed, in-table positions changed
    written = {(int(bt[p // 8]), p % 8) for p in pos.tolist() if p // 8 < bt.shape[0]}
    for pb in range(cache.shape[0]):
        for off in range(8):
            if (pb, off) not in written:
                assert torch.equal(kv[pb, :, :, off], cache[pb, :, :, off])


def check_qkv_projection_rope(impl) -> None:
    """RoPE at the new positions: Q and K equal the reference suite's own test rotation
    (apply_rope_from_scratch, fp32) applied to the unrotated fp32 projection, then rounded;
    V is not rotated."""
    h, hkv, d, hidden = 4, 2, 16, 32
    x, pos, bt, cache = _proj_case(90, h, hkv, d, hidden, seq=60, nb=8)
    w = _randn((h * d + 2 * hkv * d, hidden), 91, torch.bfloat16)
    plain_kv = cache.clone()
    plain = impl.qkv_project_paged(x, w, pos, plain_kv, bt, h, hkv, d)
    rope_kv = cache.clone()
    q = impl.qkv_project_paged(x, w, pos, rope_kv, bt, h, hkv, d, rope_base=500.0)
    xf = x[pos.long()].float()
    proj = torch.nn.functional.linear(xf, w.float())
    qf, kf = h * d, hkv * d
    q32 = proj[:, :qf].reshape(-1, h, d).permute(1, 0, 2)      # [H, R, D]: row i = pos[i]
    k32 = proj[:, qf:qf + kf].reshape(-1, hkv, d).permute(1, 0, 2)
    want_q = apply_rope_from_scratch(q32, pos.tolist(), d, 500.0).permute(1, 0, 2)
    want_k = apply_rope_from_scratch(k32, pos.tolist(), d, 500.0).permute(1, 0, 2)
    assert torch.equal(q, want_q.to(torch.bfloat16))
    for r, p in enumerate(pos.tolist()):
        pb, off = int(bt[p // 8]), p % 8
        assert torch.equal(rope_kv[pb, 0, :, off], want_k[r].to(torch.bfloat16))
        assert torch.equal(rope_kv[pb, 1, :, off], plain_kv[pb, 1, :, off])
    assert not torch.equal(q, plain)


ALL_CHECKS = [
    check_rope_reference_cases,
    check_rope_paged_reference_cases,
    check_nope_reference_cases,
    check_nope_sequential_v,
    check_apply_rope_delta,
    check_rope_golden,
    check_rope_invariants,
    check_scatter_reference_cases,
    check_scatter_golden,
    check_attention_reference_cases,
    check_attention_golden,
    check_gqa_matches_dense,
    check_projection_and_prefill,
    check_partial_prefill_selector_closed_form,
    check_partial_prefill_float64,
    check_composite_concatenation,
    check_composite_rope_concatenation,
    check_qkv_projection_mha,
    check_qkv_projection_layout,
    check_qkv_projection_rope,
]
