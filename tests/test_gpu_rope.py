"""GPU parity: RoPE delta correction family against the oracle.

Tolerances: fp32 within 1e-5 relative (1e-6 absolute floor); bf16 / fp16 within one ulp.
Cases restate synapse_kv_connector/tests/test_rope_correction.py and add seeded random,
duplicate-position, layout and full-size cases.
"""

from __future__ import annotations

import pytest
import torch

from oracle import ref_cpu as ref
from semblend_amd import rope_correction as rc
from tests.helpers import assert_bit_exact, assert_rope_close, gen, randn

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]


# ---- fused scatter + RoPE (rope_correction.py:193-282) ----

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("base", [500.0, 10000.0, 1e6])
def test_scatter_paged_random(dev, dtype, base):
    nb, h, bs, d = 64, 4, 16, 128
    kv = randn((nb, 2, h, bs, d), dtype, 1)
    donor = randn((2, h, 768, d), dtype, 2)
    bt = torch.randperm(nb, generator=gen(3))[:48].to(torch.int32)
    g = gen(4)
    tp = torch.randperm(768, generator=g)[:500].to(torch.int32)
    dp = (tp.long() + torch.randint(-300, 300, (500,), generator=g)).clamp(0, 767).to(torch.int32)
    want = ref.rope_correct_scatter_paged(kv.clone(), donor, bt, dp, tp, rope_base=base)
    got = rc.rope_correct_scatter_paged(kv.to(dev), donor.to(dev), bt.to(dev), dp.to(dev),
                                        tp.to(dev), rope_base=base)
    assert_bit_exact(got[:, 1], want[:, 1])  # V copied bit-exact
    assert_rope_close(got, want)


def test_scatter_paged_reference_cases(dev):
    """V unchanged / K corrected (test_rope_correction.py:162-233), fp32, head_dim 64."""
    nb, h, bs, d = 4, 2, 16, 64
    kv = torch.zeros((nb, 2, h, bs, d))
    donor = randn((2, h, 32, d), torch.float32, 5)
    bt = torch.arange(nb, dtype=torch.int32)
    dp = torch.tensor([0, 1, 2, 3], dtype=torch.int32)
    tp = torch.tensor([5, 10, 15, 7], dtype=torch.int32)
    want = ref.rope_correct_scatter_paged(kv.clone(), donor, bt, dp, tp)
    got = rc.rope_correct_scatter_paged(kv.to(dev), donor.to(dev), bt.to(dev), dp.to(dev),
                                        tp.to(dev))
    assert_rope_close(got, want)
    for dd, tt in zip(dp.tolist(), tp.tolist()):
        assert_bit_exact(got[tt // bs, 1, :, tt % bs], donor[1, :, dd])


def test_scatter_paged_large_delta_7b(dev):
    """Full 7B layer (cache [2048,2,4,16,128] bf16, theta 1e6) with chunk-constant deltas
    up to +-2048: angles reach 2048 rad at inv_freq[0] = 1."""
    kv = randn((2048, 2, 4, 16, 128), torch.bfloat16, 6)
    donor = randn((2, 4, 16384, 128), torch.bfloat16, 7)
    bt = torch.randperm(2048, generator=gen(8))[:1024].to(torch.int32)
    g = gen(9)
    t = torch.arange(4096, 4096 + 6000)
    delta = torch.randint(-2048, 2049, (t.shape[0] // 256 + 1,), generator=g)[t // 256 - 16]
    dp = (t - delta).to(torch.int32)
    tp = t.to(torch.int32)
    want = ref.rope_correct_scatter_paged(kv.clone(), donor, bt, dp, tp, rope_base=1e6)
    got = rc.rope_correct_scatter_paged(kv.to(dev), donor.to(dev), bt.to(dev), dp.to(dev),
                                        tp.to(dev), rope_base=1e6)
    assert_rope_close(got, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_scatter_paged_layers(dev, dtype):
    L, nb, h, bs, d = 4, 32, 8, 16, 128
    kvs = [randn((nb, 2, h, bs, d), dtype, 10 + i) for i in range(L)]
    donors = [randn((2, h, 400, d), dtype, 20 + i) for i in range(L)]
    bt = torch.randperm(nb, generator=gen(30))[:25].to(torch.int32)
    g = gen(31)
    tp = torch.randperm(400, generator=g)[:300].to(torch.int32)
    dp = torch.randint(0, 400, (300,), generator=g, dtype=torch.int32)
    want = [ref.rope_correct_scatter_paged(k.clone(), dn, bt, dp, tp, rope_base=5e5)
            for k, dn in zip(kvs, donors)]
    kd = [k.to(dev) for k in kvs]
    rc.rope_correct_scatter_paged_layers(kd, [dn.to(dev) for dn in donors], bt.to(dev),
                                         dp.to(dev), tp.to(dev), rope_base=5e5)
    for g_, w in zip(kd, want):
        assert_rope_close(g_, w)


# ---- rope_correct_k (rope_correction.py:336-399) ----

@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_correct_k_3d_4d(dev, dtype):
    k3 = randn((4, 300, 128), dtype, 40)
    g = gen(41)
    dp = torch.randperm(300, generator=g)[:200].to(torch.int32)
    tp = torch.randint(0, 5000, (200,), generator=g, dtype=torch.int32)
    want = ref.rope_correct_k(k3, dp, tp, head_dim=128, rope_base=1e6)
    got = rc.rope_correct_k(k3.to(dev), dp.to(dev), tp.to(dev), head_dim=128, rope_base=1e6)
    assert_rope_close(got, want)
    k4 = randn((3, 2, 100, 64), dtype, 42)
    want4 = ref.rope_correct_k(k4, dp[:50] % 100, tp[:50], head_dim=64)
    got4 = rc.rope_correct_k(k4.to(dev), (dp[:50] % 100).to(dev), tp[:50].to(dev), head_dim=64)
    assert_rope_close(got4, want4, composed=True)  # dp % 100 repeats positions


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_correct_k_duplicate_donor_positions(dev, dtype):
    """A row named by several pairs is rotated once per pair, in order, with a rounding to
    the dtype after each pair (the reference's sequential loop)."""
    k = randn((2, 16, 64), dtype, 43)
    dp = torch.tensor([3, 5, 3, 3, 9, 5], dtype=torch.int32)
    tp = torch.tensor([10, 1, 20, 7, 9, 100], dtype=torch.int32)
    want = ref.rope_correct_k(k, dp, tp, head_dim=64)
    got = rc.rope_correct_k(k.to(dev), dp.to(dev), tp.to(dev), head_dim=64)
    assert_rope_close(got, want, composed=True)
    inplace = k.to(dev)
    rc.rope_correct_k_inplace(inplace, dp.to(dev), tp.to(dev), head_dim=64)
    assert_rope_close(inplace, want, composed=True)


def test_rope_correct_k_reference_cases(dev):
    """Identity (Δ=0), exact move, negative delta and round trip
    (test_rope_correction.py:37-160, :294-323)."""
    k = randn((4, 8, 128), torch.float16, 44)
    pos = torch.tensor([0, 3, 7], dtype=torch.int32)
    got = rc.rope_correct_k(k.to(dev), pos.to(dev), pos.to(dev), head_dim=128)
    assert_bit_exact(got, k)
    k2 = randn((2, 10, 64), torch.float32, 45)
    s1 = rc.rope_correct_k(k2.to(dev), torch.tensor([3], dtype=torch.int32, device=dev),
                           torch.tensor([8], dtype=torch.int32, device=dev), head_dim=64)
    s2 = rc.rope_correct_k(s1, torch.tensor([3], dtype=torch.int32, device=dev),
                           torch.tensor([-2], dtype=torch.int32, device=dev), head_dim=64)
    torch.testing.assert_close(s2.cpu(), k2, atol=1e-5, rtol=1e-5)


def test_rope_correct_k_full_size_7b_inplace(dev):
    """The 7B RoPE workload: K [28, 4, 8192, 128] bf16, theta 1e6, delta constant per
    256-token chunk in [-2048, 2048]. Every position of every layer and head is compared
    with the oracle; then R(-delta) must undo R(delta) within the bf16 rounding of two
    passes."""
    k = randn((28, 4, 8192, 128), torch.bfloat16, 46)
    deltas = torch.randint(-2048, 2049, (32,), generator=gen(47))
    d = torch.arange(8192)
    t = d + deltas[d // 256]
    dd, td = d.to(torch.int32).to(dev), t.to(torch.int32).to(dev)
    kd = k.to(dev)
    rc.rope_correct_k_inplace(kd, dd, td, head_dim=128, rope_base=1e6)
    want = ref.rope_correct_k(k, d.to(torch.int32), t.to(torch.int32), head_dim=128,
                              rope_base=1e6)
    stats = assert_rope_close(kd, want)
    print(f"\n[rope 7B full] {stats}", flush=True)
    del want
    # undo: rotate the same rows (at the donor positions) by -delta
    rc.rope_correct_k_inplace(kd, dd, 2 * dd - td, head_dim=128, rope_base=1e6)
    err = (kd.float() - k.to(dev).float()).abs()
    assert float(err.max()) <= 0.07, float(err.max())  # two bf16 roundings of |x| <= ~6


@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_correct_k_distinct_donors(dev, dtype):
    """The one-launch form for distinct donor positions (shuffled pair order, a donor out of
    range skipped) lands the same bits as the indexed in-place form, and matches the oracle."""
    k = randn((3, 4, 600, 64), dtype, 49)
    g = gen(50)
    dp = torch.randperm(600, generator=g)[:450].to(torch.int32)
    dp[7] = 600  # out of range: skipped by both forms (and by the oracle)
    tp = torch.randint(-3000, 3000, (450,), generator=g, dtype=torch.int32)
    want = ref.rope_correct_k(k, dp, tp, head_dim=64, rope_base=1e4)
    a = k.to(dev)
    rc.rope_correct_k_inplace(a, dp.to(dev), tp.to(dev), head_dim=64, rope_base=1e4)
    b = k.to(dev)
    rc.rope_correct_k_inplace(b, dp.to(dev), tp.to(dev), head_dim=64, rope_base=1e4,
                              distinct_donors=True)
    assert_bit_exact(b, a.cpu())
    assert_rope_close(b, want)
    # 3-D input
    c = k[0].to(dev)
    rc.rope_correct_k_inplace(c, dp.to(dev), tp.to(dev), head_dim=64, rope_base=1e4,
                              distinct_donors=True)
    assert_bit_exact(c, b[0].cpu())


def test_rope_correct_k_distinct_full_size_7b(dev):
    """The 7B RoPE workload in its one-launch form equals the indexed form bit for bit."""
    k = randn((28, 4, 8192, 128), torch.bfloat16, 56)
    deltas = torch.randint(-2048, 2049, (32,), generator=gen(57))
    d = torch.arange(8192)
    t = d + deltas[d // 256]
    dd, td = d.to(torch.int32).to(dev), t.to(torch.int32).to(dev)
    a = k.to(dev)
    rc.rope_correct_k_inplace(a, dd, td, head_dim=128, rope_base=1e6)
    b = k.to(dev)
    rc.rope_correct_k_inplace(b, dd, td, head_dim=128, rope_base=1e6, distinct_donors=True)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_rope_bar_clause_statistics(dev, capsys):
    """How the bf16 outputs of the fused RoPE scatter meet the bar on one full Qwen2.5-7B
    layer (13926 pairs, 4 heads, deltas up to 2048, theta 1e6): most are bit-identical to the
    oracle, the rest one ulp apart; the pair-norm clause, which covers results that cancel far
    below their pair's norm, is needed by a vanishing fraction."""
    import bench

    g = torch.Generator("cpu").manual_seed(0)
    torch.randint(-2048, 2049, (32,), generator=g)
    pos_r = bench.recompute_positions(g)
    perm = torch.randperm(64, generator=g)
    t = torch.arange(16384)
    dpos = perm[t // 256] * 256 + t % 256
    keep = torch.ones(16384, dtype=torch.bool)
    keep[pos_r.long()] = False
    dp, tp = dpos[keep].to(torch.int32), t[keep].to(torch.int32)
    bt = torch.randperm(2048, generator=g)[:1024].to(torch.int32)
    kv = torch.zeros((2048, 2, 4, 16, 128), dtype=torch.bfloat16)
    donor = randn((2, 4, 16384, 128), torch.bfloat16, 70)
    got = rc.rope_correct_scatter_paged(kv.to(dev), donor.to(dev), bt.to(dev), dp.to(dev),
                                        tp.to(dev), rope_base=1e6).cpu()
    want = ref.rope_correct_scatter_paged(kv.clone(), donor, bt, dp, tp, rope_base=1e6)
    slots = bt.long()
    stats = assert_rope_close(got[slots, 0], want[slots, 0])
    with capsys.disabled():
        print(f"\n[rope bar] 7B layer, bf16 K: {stats}")
    assert stats["exact"] + stats["within_1ulp"] + stats["norm_only"] == stats["total"]
    assert stats["norm_only"] <= 1e-4 * stats["total"]
    # the same layer in fp32: how many elements pass only by the 0.1 |pair| floor
    kv32 = torch.zeros((2048, 2, 4, 16, 128), dtype=torch.float32)
    donor32 = randn((2, 4, 16384, 128), torch.float32, 70)
    got = rc.rope_correct_scatter_paged(kv32.to(dev), donor32.to(dev), bt.to(dev), dp.to(dev),
                                        tp.to(dev), rope_base=1e6).cpu()
    want = ref.rope_correct_scatter_paged(kv32.clone(), donor32, bt, dp, tp, rope_base=1e6)
    stats = assert_rope_close(got[slots, 0], want[slots, 0])
    with capsys.disabled():
        print(f"[rope bar] 7B layer, fp32 K: {stats}")
    assert stats["exact"] + stats["within_rel"] + stats["floor_only"] == stats["total"]
    assert stats["floor_only"] <= 1e-4 * stats["total"]


# ---- apply_rope_delta_inplace (rope_correction.py:699-783) ----

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("layout", ["standard", "vllm"])
def test_apply_rope_delta_inplace(dev, dtype, layout):
    nb, h, bs, d = 12, 4, 16, 128
    if layout == "standard":
        kv = randn((nb, 2, h, bs, d), dtype, 50)
    else:
        kv = randn((2, nb, bs, h, d), dtype, 50)
    bt = torch.randperm(nb, generator=gen(51))[:8].to(torch.int32)
    positions = [0, 5, 17, 17, 40, 127, 128, 300, -1, 64]  # dup, past-table, negative
    want = kv.clone()
    n_ref = ref.apply_rope_delta_inplace(want, bt, positions, 37, rope_base=1e6)
    kd = kv.to(dev)
    n_got = rc.apply_rope_delta_inplace(kd, bt.to(dev), positions, 37, rope_base=1e6)
    assert n_got == n_ref
    assert_rope_close(kd, want)
    assert rc.apply_rope_delta_inplace(kd, bt.to(dev), positions, 0) == 0
    assert rc.apply_rope_delta_inplace(kd, bt.to(dev), [], 5) == 0


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("layout", ["standard", "vllm"])
@pytest.mark.parametrize("n", [7, 256, 400])
def test_apply_rope_delta_host_and_device_positions(dev, dtype, layout, n):
    """The two C entries behind apply_rope_delta_inplace: positions by value in the launch
    (host arrays, at most SB_INLINE_POSITIONS_MAX) and positions in device memory give the
    same bits, with and without repeats; the Python function picks the first for short lists
    and the second for longer ones (n = 300), and both meet the oracle."""
    from semblend_amd import _lib
    nb, h, bs, d = 40, 2, 16, 64
    shape = (nb, 2, h, bs, d) if layout == "standard" else (2, nb, bs, h, d)
    kv = randn(shape, dtype, 70 + n)
    bt = torch.randperm(nb, generator=gen(71))[:32].to(torch.int32)
    g = gen(72 + n)
    pos = torch.randperm(32 * bs, generator=g)[:n].tolist()
    if n != 256:  # 256: exactly the most positions one launch carries, no repeats
        q = max(n // 4, 1)
        pos[:q] = pos[q: 2 * q]  # repeats
    want = kv.clone()
    n_ref = ref.apply_rope_delta_inplace(want, bt, pos, -45, rope_base=1e6)
    got = kv.to(dev)
    assert rc.apply_rope_delta_inplace(got, bt.to(dev), pos, -45, rope_base=1e6) == n_ref
    assert_bit_exact(got[:, 1] if layout == "standard" else got[1],
                     want[:, 1] if layout == "standard" else want[1])
    assert_rope_close(got, want)
    counts, _ = rc._rotation_counts(pos, bs, bt.shape[0])
    keys, reps = list(counts.keys()), list(counts.values())
    if len(keys) > _lib.SB_INLINE_POSITIONS_MAX:
        with pytest.raises(RuntimeError, match="SB_INLINE_POSITIONS_MAX"):
            _lib.call("sb_apply_rope_delta_inplace_host", got.data_ptr(), 0,
                      _lib.i32_array(keys), None, len(keys), 1, 0, h, bs, d, nb, 32,
                      _lib.i64_array([1, 1, 1, 1]), _lib.dtype_code(got), 0)
        return
    st = got.stride()
    kst = (st[0], st[2], st[3], st[4]) if layout == "standard" else (st[1], st[3], st[2], st[4])
    inv = rc.inv_freq_table(1e6, d, dev)
    btd = bt.to(dev)
    results = []
    for host in (True, False):
        for with_rep in (True, False):
            x = kv.to(dev)
            args_tail = (len(keys), -45, inv.data_ptr(), h, bs, d, nb, 32, _lib.i64_array(kst),
                         _lib.dtype_code(x), _lib.stream_handle(dev))
            if host:
                _lib.call("sb_apply_rope_delta_inplace_host", x.data_ptr(), btd.data_ptr(),
                          _lib.i32_array(keys), _lib.i32_array(reps) if with_rep else None,
                          *args_tail)
            else:
                kd = torch.tensor(keys, dtype=torch.int32, device=dev)
                rd = torch.tensor(reps, dtype=torch.int32, device=dev)
                _lib.call("sb_apply_rope_delta_inplace", x.data_ptr(), btd.data_ptr(),
                          kd.data_ptr(), rd.data_ptr() if with_rep else None, *args_tail)
            results.append(x.cpu())
    assert_bit_exact(results[0], results[2])  # with repeats: host == device positions
    assert_bit_exact(results[1], results[3])  # once each
    assert_bit_exact(results[0], got)


def test_apply_rope_delta_round_trip(dev):
    """Δ then -Δ is the identity up to rounding (semblend_connector.py:609-616 relies on it)."""
    kv = randn((8, 2, 4, 16, 64), torch.float32, 52)
    bt = torch.arange(8, dtype=torch.int32)
    kd = kv.to(dev)
    pos = list(range(0, 128, 3))
    rc.apply_rope_delta_inplace(kd, bt.to(dev), pos, 1234)
    rc.apply_rope_delta_inplace(kd, bt.to(dev), pos, -1234)
    torch.testing.assert_close(kd.cpu(), kv, atol=2e-6, rtol=2e-6)


# ---- permutations (rope_correction.py:407-476, :599-697) ----

@pytest.mark.parametrize("dtype", DTYPES)
def test_permute_paged_kv_with_rope(dev, dtype):
    nb, h, bs, d = 10, 2, 16, 64
    kv = randn((nb, 2, h, bs, d), dtype, 60)
    bt = torch.randperm(nb, generator=gen(61))[:8].to(torch.int32)
    g = gen(62)
    src = torch.randperm(128, generator=g)[:90].tolist()
    tgt = torch.randperm(128, generator=g)[:90].tolist()
    perm = list(zip(src, tgt)) + [(0, 1), (1, 0)]
    perm = list({t: (s, t) for s, t in perm}.values())  # distinct targets
    want = kv.clone()
    ref.permute_paged_kv_with_rope(want, bt, perm, rope_base=1e6)
    kd = kv.to(dev)
    rc.permute_paged_kv_with_rope(kd, bt.to(dev), perm, rope_base=1e6)
    assert_bit_exact(kd[:, 1], want[:, 1])
    assert_rope_close(kd, want)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_nope_permute_paged_kv(dev, dtype):
    nb, h, bs, d = 10, 4, 16, 128
    kv = randn((nb, 2, h, bs, d), dtype, 63)
    bt = torch.randperm(nb, generator=gen(64))[:8].to(torch.int32)
    # chains and a swap, so the sequential V copies of the reference matter
    perm = [(2, 10), (10, 30), (30, 2), (5, 6), (6, 5), (40, 41), (77, 100), (100, 3)]
    want = kv.clone()
    ref.nope_permute_paged_kv(want, bt, perm)
    kd = kv.to(dev)
    rc.nope_permute_paged_kv(kd, bt.to(dev), perm)
    assert_bit_exact(kd[:, 1], want[:, 1])
    assert_rope_close(kd, want)
