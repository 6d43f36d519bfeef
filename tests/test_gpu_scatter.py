"""GPU parity: donor-KV scatter (flat, paged, multi-layer) is bit-exact against the oracle.

Cases restate synapse_kv_connector/tests/test_triton_kernels.py:79-302 and add seeded random
and full-size cases (Qwen2.5-7B KV shape: 4 KV heads x 128, bf16, block size 16).
"""

from __future__ import annotations

import pytest
import torch

import bench
from oracle import ref_cpu as ref
from semblend_amd import rope_correction as rc
from semblend_amd import triton_kernels as tk
from tests.helpers import assert_bit_exact, assert_rope_close, gen, randn

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16, torch.float32]


# ---- flat scatter (test_triton_kernels.py:79-168) ----

def test_flat_basic(dev):
    target = torch.zeros((2, 2, 4, 16, 32), dtype=torch.float16)
    donor = randn((2, 2, 4, 8, 32), torch.float16, 1)
    dp = torch.tensor([0, 2, 4, 6], dtype=torch.int32)
    tp = torch.tensor([1, 3, 7, 12], dtype=torch.int32)
    got = tk.scatter_donor_kv(target.to(dev), donor.to(dev), dp.to(dev), tp.to(dev))
    assert_bit_exact(got, ref.scatter_donor_kv(target.clone(), donor, dp, tp))
    for p in (0, 2, 4):
        assert torch.all(got[:, :, :, p].cpu() == 0)


def test_flat_empty_and_single(dev):
    target = torch.zeros((1, 2, 2, 8, 16), dtype=torch.float16, device=dev)
    donor = randn((1, 2, 2, 4, 16), torch.float16, 2).to(dev)
    empty = torch.zeros(0, dtype=torch.int32, device=dev)
    assert torch.all(tk.scatter_donor_kv(target, donor, empty, empty) == 0)
    t1 = torch.zeros((1, 2, 1, 4, 8), dtype=torch.float16, device=dev)
    d1 = randn((1, 2, 1, 2, 8), torch.float16, 3).to(dev)
    tk.scatter_donor_kv(t1, d1, torch.tensor([1], dtype=torch.int32, device=dev),
                        torch.tensor([3], dtype=torch.int32, device=dev))
    assert_bit_exact(t1[0, :, 0, 3], d1[0, :, 0, 1])


@pytest.mark.parametrize("dtype", DTYPES)
def test_flat_full_and_multilayer(dev, dtype):
    donor = randn((8, 2, 4, 64, 64), dtype, 4)
    target = torch.zeros((8, 2, 4, 64, 64), dtype=dtype)
    pos = torch.arange(64, dtype=torch.int32)
    got = tk.scatter_donor_kv(target.to(dev), donor.to(dev), pos.to(dev), pos.to(dev))
    assert_bit_exact(got, donor)


@pytest.mark.parametrize("dtype", DTYPES)
def test_flat_random_with_out_of_range(dev, dtype):
    g = gen(5)
    donor = randn((3, 2, 5, 40, 96), dtype, 6)
    target = randn((3, 2, 5, 50, 96), dtype, 7)
    dp = torch.randint(-3, 45, (60,), generator=g, dtype=torch.int32)
    tp = torch.randperm(55, generator=g)[:60].to(torch.int32) - 2  # unique targets, some OOB
    dp = dp[: tp.shape[0]]
    got = tk.scatter_donor_kv(target.to(dev), donor.to(dev), dp.to(dev), tp.to(dev))
    assert_bit_exact(got, ref.scatter_donor_kv(target.clone(), donor, dp, tp))


# ---- paged scatter (test_triton_kernels.py:176-302) ----

def test_paged_reference_cases(dev):
    kv = torch.zeros((8, 2, 2, 4, 16), dtype=torch.float16)
    donor = randn((2, 2, 8, 16), torch.float16, 8)
    bt = torch.tensor([3, 5], dtype=torch.int32)
    dp = torch.tensor([0, 4], dtype=torch.int32)
    tp = torch.tensor([1, 5], dtype=torch.int32)
    got = tk.scatter_donor_kv_paged(kv.to(dev), donor.to(dev), bt.to(dev), dp.to(dev),
                                    tp.to(dev)).cpu()
    assert_bit_exact(got[3, :, :, 1], donor[:, :, 0])
    assert_bit_exact(got[5, :, :, 1], donor[:, :, 4])
    # same block, several offsets
    kv2 = torch.zeros((4, 2, 2, 8, 16), dtype=torch.float16)
    got2 = tk.scatter_donor_kv_paged(
        kv2.to(dev), donor.to(dev), torch.tensor([2], dtype=torch.int32, device=dev),
        torch.tensor([0, 1, 2], dtype=torch.int32, device=dev),
        torch.tensor([0, 3, 7], dtype=torch.int32, device=dev)).cpu()
    for d, t in zip([0, 1, 2], [0, 3, 7]):
        assert_bit_exact(got2[2, :, :, t], donor[:, :, d])
    # out-of-range logical block skipped
    kv3 = torch.zeros((4, 2, 1, 4, 8), dtype=torch.float16)
    d3 = randn((2, 1, 4, 8), torch.float16, 9)
    got3 = tk.scatter_donor_kv_paged(
        kv3.to(dev), d3.to(dev), torch.tensor([1], dtype=torch.int32, device=dev),
        torch.tensor([0, 1], dtype=torch.int32, device=dev),
        torch.tensor([2, 8], dtype=torch.int32, device=dev)).cpu()
    assert_bit_exact(got3[1, :, :, 2], d3[:, :, 0])
    got3[1, :, :, 2] = 0
    assert torch.all(got3 == 0)
    # empty
    empty = torch.zeros(0, dtype=torch.int32, device=dev)
    z = torch.zeros((4, 2, 2, 4, 8), dtype=torch.float16, device=dev)
    zd = randn((2, 2, 4, 8), torch.float16, 10).to(dev)
    bt0 = torch.tensor([0, 1], dtype=torch.int32, device=dev)
    assert torch.all(tk.scatter_donor_kv_paged(z, zd, bt0, empty, empty) == 0)


def _chunk_pairs(seq_len: int, chunk: int, n_drop: int, seed: int):
    """Donor chunks reused in shuffled order: d = chunk*pi(c)+j -> t = chunk*c+j, with n_drop
    random target positions left out (they are recomputed)."""
    g = gen(seed)
    n_chunks = seq_len // chunk
    perm = torch.randperm(n_chunks, generator=g)
    t = torch.arange(seq_len)
    d = perm[t // chunk] * chunk + t % chunk
    keep = torch.ones(seq_len, dtype=torch.bool)
    keep[torch.randperm(seq_len, generator=g)[:n_drop]] = False
    return d[keep].to(torch.int32), t[keep].to(torch.int32)


@pytest.mark.parametrize("dtype", DTYPES)
def test_paged_random(dev, dtype):
    nb, h, bs, d = 96, 3, 16, 64
    kv = randn((nb, 2, h, bs, d), dtype, 10)
    donor = randn((2, h, 1024, d), dtype, 11)
    bt = torch.randperm(nb, generator=gen(12))[:64].to(torch.int32)
    dp, tp = _chunk_pairs(1024, 256, 150, 13)
    bt[5] = 1000  # an invalid physical block: its 16 target positions are skipped
    got = tk.scatter_donor_kv_paged(kv.to(dev), donor.to(dev), bt.to(dev), dp.to(dev),
                                    tp.to(dev))
    assert_bit_exact(got, ref.scatter_donor_kv_paged(kv.clone(), donor, bt, dp, tp))


def test_paged_strided_layout(dev):
    """A cache whose logical [NB, 2, H, bs, D] view has non-standard strides (allocated as
    [2, NB, bs, H, D], the vLLM flash-attn order)."""
    nb, h, bs, d = 32, 4, 16, 128
    base = randn((2, nb, bs, h, d), torch.bfloat16, 14)
    view_cpu = base.permute(1, 0, 3, 2, 4)
    donor = randn((2, h, 256, d), torch.bfloat16, 15)
    bt = torch.randperm(nb, generator=gen(16))[:16].to(torch.int32)
    dp, tp = _chunk_pairs(256, 64, 20, 17)
    want = ref.scatter_donor_kv_paged(view_cpu.clone(), donor, bt, dp, tp)
    base_dev = base.to(dev)
    view = base_dev.permute(1, 0, 3, 2, 4)
    tk.scatter_donor_kv_paged(view, donor.to(dev), bt.to(dev), dp.to(dev), tp.to(dev))
    assert_bit_exact(view, want)


def test_paged_full_size_7b_layer(dev):
    """One layer of the 7B scatter workload: cache [2048, 2, 4, 16, 128] bf16, 16384-token
    target, 64 shuffled 256-token donor chunks, 2458 recomputed positions left unwritten."""
    kv = randn((2048, 2, 4, 16, 128), torch.bfloat16, 20)
    donor = randn((2, 4, 16384, 128), torch.bfloat16, 21)
    bt = torch.randperm(2048, generator=gen(22))[:1024].to(torch.int32)
    dp, tp = _chunk_pairs(16384, 256, 2458, 23)
    assert dp.shape[0] == 13926
    want = ref.scatter_donor_kv_paged(kv.clone(), donor, bt, dp, tp)
    got = tk.scatter_donor_kv_paged(kv.to(dev), donor.to(dev), bt.to(dev), dp.to(dev),
                                    tp.to(dev))
    assert_bit_exact(got, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_paged_layers_matches_per_layer(dev, dtype):
    L, nb, h, bs, d = 5, 40, 2, 16, 128
    kvs = [randn((nb, 2, h, bs, d), dtype, 30 + i) for i in range(L)]
    donors = [randn((2, h, 512, d), dtype, 40 + i) for i in range(L)]
    bt = torch.randperm(nb, generator=gen(50))[:32].to(torch.int32)
    dp, tp = _chunk_pairs(512, 128, 70, 51)
    want = [ref.scatter_donor_kv_paged(k.clone(), dn, bt, dp, tp) for k, dn in zip(kvs, donors)]
    kvs_dev = [k.to(dev) for k in kvs]
    tk.scatter_donor_kv_paged_layers(kvs_dev, [dn.to(dev) for dn in donors], bt.to(dev),
                                     dp.to(dev), tp.to(dev))
    for g, w in zip(kvs_dev, want):
        assert_bit_exact(g, w)


@pytest.mark.parametrize("rope", [False, True])
def test_paged_layers_repeated_donor_rows(dev, rope):
    """Donor rows that feed several targets (chunk deltas whose donor windows overlap): the
    cached-load policy, the nontemporal one and the automatic choice give the same bits, and
    every layer meets the oracle (copies bit-exact, rotated K within the RoPE bar)."""
    L, nb, h, bs, d = 3, 48, 2, 16, 128
    kvs = [randn((nb, 2, h, bs, d), torch.bfloat16, 300 + i) for i in range(L)]
    donors = [randn((2, h, 256, d), torch.bfloat16, 310 + i) for i in range(L)]
    bt = torch.randperm(nb, generator=gen(320))[:40].to(torch.int32)
    tp = torch.arange(0, 600, dtype=torch.int32)
    dp = (tp % 200 + 20).to(torch.int32)  # each donor row is read by three targets
    if rope:
        want = [ref.rope_correct_scatter_paged(k.clone(), dn, bt, dp, tp, 5e5)
                for k, dn in zip(kvs, donors)]
    else:
        want = [ref.scatter_donor_kv_paged(k.clone(), dn, bt, dp, tp)
                for k, dn in zip(kvs, donors)]
    dd = [dn.to(dev) for dn in donors]
    results = {}
    for repeated in (False, True, None):
        got = [k.to(dev) for k in kvs]
        if rope:
            call = rc.prepare_scatter_paged_layers(got, dd, bt.to(dev), dp.to(dev),
                                                   tp.to(dev), 5e5, repeated_donor_rows=repeated)
            assert (call.args[-1] == 1) == (repeated is not False)
            call()
        else:
            tk.scatter_donor_kv_paged_layers(got, dd, bt.to(dev), dp, tp,
                                             repeated_donor_rows=repeated)
        results[repeated] = [g.cpu() for g in got]
    for repeated in (True, None):
        for a, b in zip(results[repeated], results[False]):
            assert_bit_exact(a, b)
    for g, w in zip(results[False], want):
        if rope:
            assert_bit_exact(g[:, 1], w[:, 1])
            assert_rope_close(g, w)
        else:
            assert_bit_exact(g, w)


def test_paged_layers_full_size_7b(dev):
    """The timed 28-layer launch of the 7B scatter workload (caches [2048, 2, 4, 16, 128]
    bf16, donors [2, 4, 16384, 128]) with the pairs bench.py builds: 64 donor chunks reused
    in shuffled order, minus the structured recompute set (the first 256 tokens, two whole
    chunks, the rest scattered): 13926 pairs. Every layer equals the oracle's scatter of
    that layer bit for bit, and the single-layer entry lands the same bits."""
    L = 28
    g = gen(60)
    pos_r = bench.recompute_positions(g)
    perm = torch.randperm(64, generator=g)
    t = torch.arange(16384)
    d = perm[t // 256] * 256 + t % 256
    keep = torch.ones(16384, dtype=torch.bool)
    keep[pos_r.long()] = False
    dp, tp = d[keep].to(torch.int32), t[keep].to(torch.int32)
    assert dp.shape[0] == 13926
    bt = torch.randperm(2048, generator=g)[:1024].to(torch.int32)
    kvs = [randn((2048, 2, 4, 16, 128), torch.bfloat16, 100 + i).to(dev) for i in range(L)]
    donors = [randn((2, 4, 16384, 128), torch.bfloat16, 200 + i).to(dev) for i in range(L)]
    btd, dpd, tpd = bt.to(dev), dp.to(dev), tp.to(dev)
    tk.scatter_donor_kv_paged_layers(kvs, donors, btd, dpd, tpd)
    for layer in range(L):
        kv0 = randn((2048, 2, 4, 16, 128), torch.bfloat16, 100 + layer)
        single = tk.scatter_donor_kv_paged(kv0.to(dev), donors[layer], btd, dpd, tpd)
        assert torch.equal(kvs[layer].view(torch.int16), single.view(torch.int16))
        del single
        want = ref.scatter_donor_kv_paged(kv0, donors[layer].cpu(), bt, dp, tp)
        assert_bit_exact(kvs[layer], want)


def test_cpu_tensors_rejected():
    kv = torch.zeros((2, 2, 1, 4, 8))
    with pytest.raises(RuntimeError, match="device tensors"):
        tk.scatter_donor_kv_paged(kv, torch.zeros((2, 1, 4, 8)), torch.tensor([0]),
                                  torch.tensor([0]), torch.tensor([0]))


# ---- the flat copy the movers' bandwidth is compared with ----

@pytest.mark.parametrize("nbytes", [16, 4096 + 16, (1 << 20) + 48, 64 << 20])
def test_device_copy_bytes(dev, nbytes):
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, generator=gen(31)).to(dev)
    dst = torch.zeros_like(src)
    from semblend_amd import _lib
    _lib.device_copy(dst, src)
    torch.cuda.synchronize()
    assert torch.equal(dst, src)


def test_device_copy_rejects_unaligned(dev):
    from semblend_amd import _lib
    a = torch.zeros(64, dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError, match="multiple of 16"):
        _lib.device_copy(a[:40], a[16:56])
    with pytest.raises(RuntimeError, match="aligned"):
        _lib.device_copy(a[1:17], a[32:48])
