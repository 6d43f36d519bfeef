"""GPU parity: the chunked host-to-device donor load with RoPE on the fly.

The streamed result must equal, bit for bit, the one-shot fused RoPE scatter from the whole
donor already on the device (same kernel arithmetic, only the source rows are staged), and
one layer is checked against the oracle. Chunks are LMCache-layout [2, L, T, H*D] tensors
in pinned host memory; the last chunk is partial.
"""

from __future__ import annotations

import pytest
import torch

from oracle import ref_cpu as ref
from semblend_amd import rope_correction as rc
from semblend_amd import triton_kernels as tk
from semblend_amd.loader import ChunkedKVLoader
from tests.helpers import assert_rope_close, gen, randn

pytestmark = pytest.mark.gpu


def _host_chunks(donors, chunk):
    """LMCache KV_2LTD chunks [2, L, T_c, H*D] (pinned) of per-layer donors [2, H, S, D]."""
    L = len(donors)
    _, h, s, d = donors[0].shape
    out = []
    for c0 in range(0, s, chunk):
        c1 = min(c0 + chunk, s)
        x = torch.stack([dn[:, :, c0:c1].permute(0, 2, 1, 3) for dn in donors], dim=1)
        out.append(x.reshape(2, L, c1 - c0, h * d).contiguous().pin_memory())
    return out


def _pairs(donor_len, target_len, chunk, seed, n_recompute=150):
    """Donor chunks reused in shuffled order, minus recompute positions, plus pairs past the
    donor's end (skipped)."""
    g = gen(seed)
    n = min(donor_len, target_len)
    nch = (n + chunk - 1) // chunk
    perm = torch.randperm(nch, generator=g)
    t = torch.arange(n)
    d = perm[t // chunk] * chunk + t % chunk
    keep = (d < donor_len) & (torch.rand(n, generator=g) > n_recompute / n)
    d, t = d[keep], t[keep]
    d = torch.cat([d, torch.tensor([donor_len, donor_len + 3])])
    t = torch.cat([t, torch.tensor([target_len - 1, target_len - 2])])
    return d.to(torch.int32), t.to(torch.int32)


def _setup(dtype, layers=3, h=4, donor_len=1800, seed=0):
    d = 64 if dtype == torch.float32 else 128
    donors = [randn((2, h, donor_len, d), dtype, seed + l) for l in range(layers)]
    caches = [randn((150, 2, h, 16, d), dtype, seed + 10 + l) for l in range(layers)]
    bt = torch.randperm(150, generator=gen(seed + 20))[:128].to(torch.int32)
    return donors, caches, bt


@pytest.mark.parametrize("rope", [True, False], ids=["rope", "copy"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_loader_matches_one_shot(dev, dtype, rope):
    donors, caches, bt = _setup(dtype)
    dpos, tpos = _pairs(1800, 2048, 256, 1)
    chunks = _host_chunks(donors, 256)
    assert len(chunks) == 8 and chunks[-1].shape[2] == 1800 - 7 * 256
    got = [c.to(dev) for c in caches]
    loader = ChunkedKVLoader(got, bt.to(dev), chunk_tokens=256, slots=3, rope_base=1e6)
    loader.load(chunks, dpos, tpos, rope=rope)
    want = [c.to(dev) for c in caches]
    dd = [x.to(dev) for x in donors]
    if rope:
        rc.rope_correct_scatter_paged_layers(want, dd, bt.to(dev), dpos.to(dev), tpos.to(dev),
                                             rope_base=1e6)
    else:
        tk.scatter_donor_kv_paged_layers(want, dd, bt.to(dev), dpos.to(dev), tpos.to(dev))
    for a, b in zip(got, want):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))
    # one layer against the oracle
    exp = caches[1].clone()
    if rope:
        ref.rope_correct_scatter_paged(exp, donors[1], bt, dpos, tpos, rope_base=1e6)
        assert torch.equal(got[1][:, 1].cpu().view(torch.uint8), exp[:, 1].view(torch.uint8))
        assert_rope_close(got[1][:, 0], exp[:, 0])
    else:
        ref.scatter_donor_kv_paged(exp, donors[1], bt, dpos, tpos)
        assert torch.equal(got[1].cpu().view(torch.uint8), exp.view(torch.uint8))


@pytest.mark.parametrize("slots", [1, 2])
def test_loader_ring_sizes_and_repeated_loads(dev, slots):
    """Two donors loaded one after the other through the same ring (disjoint targets), as a
    composite plan's donors would be; a ring of one slot serialises copy and scatter."""
    dtype = torch.bfloat16
    donors_a, caches, bt = _setup(dtype, donor_len=1024, seed=30)
    donors_b, _, _ = _setup(dtype, donor_len=700, seed=40)
    g = gen(41)
    targets = torch.randperm(2048, generator=g).to(torch.int32)
    ta, tb = targets[:900], targets[900:1500]
    da = torch.randint(0, 1024, (900,), generator=g).to(torch.int32)
    db = torch.randint(0, 700, (600,), generator=g).to(torch.int32)
    got = [c.to(dev) for c in caches]
    loader = ChunkedKVLoader(got, bt.to(dev), chunk_tokens=128, slots=slots, rope_base=1e4)
    loader.load(_host_chunks(donors_a, 128), da, ta)
    loader.load(_host_chunks(donors_b, 128), db, tb)
    want = [c.to(dev) for c in caches]
    for dn, d, t in ((donors_a, da, ta), (donors_b, db, tb)):
        rc.rope_correct_scatter_paged_layers(want, [x.to(dev) for x in dn], bt.to(dev),
                                             d.to(dev), t.to(dev), rope_base=1e4)
    for a, b in zip(got, want):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_loader_rejects_bad_chunks(dev):
    donors, caches, bt = _setup(torch.bfloat16, layers=2, donor_len=300)
    kv = [c.to(dev) for c in caches]
    loader = ChunkedKVLoader(kv, bt.to(dev), chunk_tokens=256)
    good = _host_chunks(donors, 256)
    d = torch.arange(10, dtype=torch.int32)
    with pytest.raises(ValueError, match="pinned"):
        loader.load([good[0].clone()], d, d)           # pageable memory
    with pytest.raises(ValueError, match="host"):
        loader.load([good[0].to(dev)], d, d)           # already on the GPU
    with pytest.raises(ValueError, match="at most"):
        loader.load([torch.zeros((2, 2, 300, 512), dtype=torch.bfloat16).pin_memory()], d, d)
    with pytest.raises(ValueError):
        loader.load([torch.zeros((2, 3, 16, 512), dtype=torch.bfloat16).pin_memory()], d, d)
    with pytest.raises(TypeError):
        loader.load([torch.zeros((2, 2, 16, 512), dtype=torch.float16).pin_memory()], d, d)


def test_loader_no_pairs_and_unread_chunks(dev):
    """A load whose pairs all lie outside the chunks changes nothing; chunks no pair reads
    are skipped (only the read chunk's rows land)."""
    donors, caches, bt = _setup(torch.bfloat16, layers=2, donor_len=600)
    kv = [c.to(dev) for c in caches]
    loader = ChunkedKVLoader(kv, bt.to(dev), chunk_tokens=256, slots=2)
    chunks = _host_chunks(donors, 256)
    loader.load(chunks, torch.tensor([700, -3], dtype=torch.int32),
                torch.tensor([1, 2], dtype=torch.int32))
    loader.load(chunks, torch.zeros(0, dtype=torch.int32), torch.zeros(0, dtype=torch.int32))
    for a, b in zip(kv, caches):
        assert torch.equal(a.cpu().view(torch.int16), b.view(torch.int16))
    d = torch.arange(300, 310, dtype=torch.int32)          # chunk 1 only
    t = torch.arange(40, 50, dtype=torch.int32)
    loader.load(chunks, d, t)
    want = [c.to(dev) for c in caches]
    rc.rope_correct_scatter_paged_layers(want, [x.to(dev) for x in donors], bt.to(dev),
                                         d.to(dev), t.to(dev), rope_base=10000.0)
    for a, b in zip(kv, want):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
