"""GPU parity: multi-donor (composite) scatter against the oracle's per-donor composition.

Donors differ in length and in strides (some are views into larger buffers); targets are
256-token-style chunks assigned to donors at random, as a composite plan does, with a few
pairs that must be skipped (unknown donor ids, donor positions past a donor's end).
V is bit-exact; K is bit-exact for plain copies and within the RoPE bar when rotated.
"""

from __future__ import annotations

import pytest
import torch

from oracle import ref_cpu as ref
from semblend_amd import rope_correction as rc
from semblend_amd import triton_kernels as tk
from semblend_amd.multi_donor import (
    MultiDonorPositionMapping,
    composite_scatter_paged,
    composite_scatter_paged_layers,
    prepare_composite_scatter_paged_layers,
)
from tests.helpers import assert_rope_close, gen, randn

pytestmark = pytest.mark.gpu


def _donor(n, h, d, dtype, seed, pad=0):
    """[2, h, n, d]; with pad > 0 a view into a longer buffer (sequence stride kept, kv and
    head strides those of the longer buffer)."""
    full = randn((2, h, n + pad, d), dtype, seed)
    return full[:, :, :n] if pad else full


def _plan(lens, nb_seq, bs, chunk, seed, skip_frac=0.2):
    """Chunk-wise owners: each target chunk is skipped or copied from a random window of a
    random donor. Returns donor_index, donor_pos, target_pos (int32) with invalid pairs
    appended (unknown donor ids, a donor position at the donor's end)."""
    g = gen(seed)
    didx, dpos, tpos = [], [], []
    n_chunks = nb_seq * bs // chunk
    for c in range(n_chunks):
        if float(torch.rand(1, generator=g)) < skip_frac:
            continue
        k = int(torch.randint(0, len(lens), (1,), generator=g))
        n = min(chunk, lens[k])
        start = int(torch.randint(0, lens[k] - n + 1, (1,), generator=g))
        didx += [k] * n
        dpos += list(range(start, start + n))
        tpos += list(range(c * chunk, c * chunk + n))
    free = sorted(set(range(nb_seq * bs)) - set(tpos))[:3]
    didx += [len(lens), -1, 0][: len(free)]
    dpos += [0, 0, lens[0]][: len(free)]
    tpos += free
    t = lambda v: torch.tensor(v, dtype=torch.int32)
    return t(didx), t(dpos), t(tpos)


def _caches(layers, nb, h, bs, d, dtype, seed):
    return [randn((nb, 2, h, bs, d), dtype, seed + l) for l in range(layers)]


def _check(got, want, rope):
    got = got.cpu()
    assert torch.equal(got[:, 1].view(torch.uint8), want[:, 1].view(torch.uint8))
    if rope:
        assert_rope_close(got[:, 0], want[:, 0])
    else:
        assert torch.equal(got[:, 0].view(torch.uint8), want[:, 0].view(torch.uint8))


@pytest.mark.parametrize("rope", [True, False], ids=["rope", "copy"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_composite_matches_oracle(dev, dtype, rope):
    layers, h, bs = 3, 4, 16
    d = 64 if dtype == torch.float32 else 128
    lens = [300, 517, 1024]
    donors = [[_donor(n, h, d, dtype, 100 * k + l, pad=40 if k == 1 else 0)
               for l in range(layers)] for k, n in enumerate(lens)]
    nb, nb_seq = 160, 128
    bt = torch.randperm(nb, generator=gen(5))[:nb_seq].to(torch.int32)
    didx, dpos, tpos = _plan(lens, nb_seq, bs, 64, 6)
    caches = _caches(layers, nb, h, bs, d, dtype, 7)
    got = [c.to(dev) for c in caches]
    composite_scatter_paged_layers(got, [[t.to(dev) for t in per] for per in donors],
                                   bt.to(dev), didx.to(dev), dpos.to(dev), tpos.to(dev),
                                   rope=rope, rope_base=1e6)
    for l in range(layers):
        want = ref.composite_scatter_paged(caches[l].clone(), [per[l] for per in donors], bt,
                                           didx, dpos, tpos, rope=rope, rope_base=1e6)
        _check(got[l], want, rope)


@pytest.mark.parametrize("rope", [True, False], ids=["rope", "copy"])
def test_composite_load_policy_same_bits(dev, rope):
    """Donor windows of different chunks overlap in this plan (donor rows read by several
    pairs): the cached-load policy, the nontemporal one and the choice made from host
    positions give the same bits."""
    from semblend_amd import _lib
    layers, h, bs, d, dtype = 2, 4, 16, 128, torch.bfloat16
    lens = [300, 517]
    donors = [[_donor(n, h, d, dtype, 300 + 10 * k + l).to(dev) for l in range(layers)]
              for k, n in enumerate(lens)]
    nb, nb_seq = 96, 80
    bt = torch.randperm(nb, generator=gen(8))[:nb_seq].to(torch.int32)
    didx, dpos, tpos = _plan(lens, nb_seq, bs, 64, 9, skip_frac=0.0)
    assert _lib.rows_repeat(dpos, didx)
    caches = _caches(layers, nb, h, bs, d, dtype, 11)
    outs = []
    for policy, host in ((False, False), (True, False), (None, True)):
        got = [c.to(dev) for c in caches]
        idx = (didx, dpos, tpos) if host else (didx.to(dev), dpos.to(dev), tpos.to(dev))
        composite_scatter_paged_layers(got, donors, bt.to(dev), *idx, rope=rope,
                                       rope_base=1e6, repeated_donor_rows=policy)
        outs.append([g.cpu() for g in got])
    for other in outs[1:]:
        for a, b in zip(outs[0], other):
            assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def test_composite_single_donor_equals_layers_entries(dev):
    layers, h, bs, d, dtype = 4, 4, 16, 128, torch.bfloat16
    donor = [randn((2, h, 700, d), dtype, 30 + l).to(dev) for l in range(layers)]
    bt = torch.randperm(64, generator=gen(31))[:48].to(torch.int32).to(dev)
    g = gen(32)
    tpos = torch.randperm(48 * bs, generator=g)[:600].to(torch.int32).to(dev)
    dpos = torch.randint(0, 700, (600,), generator=g).to(torch.int32).to(dev)
    didx = torch.zeros(600, dtype=torch.int32, device=dev)
    base = [randn((64, 2, h, bs, d), dtype, 33 + l).to(dev) for l in range(layers)]
    for rope in (True, False):
        a = [c.clone() for c in base]
        b = [c.clone() for c in base]
        composite_scatter_paged_layers(a, [donor], bt, didx, dpos, tpos, rope=rope,
                                       rope_base=5e5)
        if rope:
            rc.rope_correct_scatter_paged_layers(b, donor, bt, dpos, tpos, rope_base=5e5)
        else:
            tk.scatter_donor_kv_paged_layers(b, donor, bt, dpos, tpos)
        for x, y in zip(a, b):
            assert torch.equal(x.view(torch.int16), y.view(torch.int16))


def test_composite_donor_windows(dev):
    """Donor tensors that hold only a window [f, f + S) of their donor (first positions
    given) give the same bits as the whole donors: rows are read at d - f, K is rotated by
    the true t - d; pairs outside a window are skipped."""
    layers, h, bs, d, dtype = 2, 4, 16, 128, torch.bfloat16
    lens = [600, 900]
    donors = [[randn((2, h, n, d), dtype, 300 + 10 * k + l).to(dev) for l in range(layers)]
              for k, n in enumerate(lens)]
    windows = [(128, 300), (512, 256)]      # (first, rows)
    g = gen(301)
    tpos = torch.randperm(64 * bs, generator=g)[:400].to(torch.int32)
    didx = torch.randint(0, 2, (400,), generator=g).to(torch.int32)
    first = torch.tensor([w[0] for w in windows])[didx.long()]
    rows = torch.tensor([w[1] for w in windows])[didx.long()]
    inside = first + (torch.rand(400, generator=g) * rows).long()
    dpos = inside.to(torch.int32)
    dpos[:5] = first[:5].to(torch.int32) - 1                 # just before a window: skipped
    bt = torch.randperm(80, generator=gen(302))[:64].to(torch.int32).to(dev)
    base = [randn((80, 2, h, bs, d), dtype, 303 + l).to(dev) for l in range(layers)]
    got = [c.clone() for c in base]
    composite_scatter_paged_layers(
        got, [[t[:, :, f:f + n] for t in per] for per, (f, n) in zip(donors, windows)], bt,
        didx, dpos, tpos, rope=True, rope_base=1e4,
        donor_first_positions=[f for f, _ in windows])
    want = [c.clone() for c in base]
    composite_scatter_paged_layers(want, donors, bt, didx[5:], dpos[5:], tpos[5:], rope=True,
                                   rope_base=1e4)
    for a, b in zip(got, want):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_composite_many_donors_two_launches(dev):
    # 20 donors: two launches of at most 16 donors each
    layers, h, bs, d, dtype = 2, 2, 16, 64, torch.bfloat16
    lens = [40 + 3 * k for k in range(20)]
    donors = [[_donor(n, h, d, dtype, 200 + 10 * k + l) for l in range(layers)]
              for k, n in enumerate(lens)]
    bt = torch.randperm(80, generator=gen(40))[:64].to(torch.int32)
    didx, dpos, tpos = _plan(lens, 64, bs, 32, 41, skip_frac=0.1)
    caches = _caches(layers, 80, h, bs, d, dtype, 42)
    got = [c.to(dev) for c in caches]
    composite_scatter_paged_layers(got, [[t.to(dev) for t in per] for per in donors],
                                   bt.to(dev), didx, dpos, tpos, rope=True, rope_base=1e4)
    for l in range(layers):
        want = ref.composite_scatter_paged(caches[l].clone(), [per[l] for per in donors], bt,
                                           didx, dpos, tpos, rope=True, rope_base=1e4)
        _check(got[l], want, True)


def test_composite_from_mapping_vllm_layout(dev):
    """String donor ids through MultiDonorPositionMapping, into a vLLM flash-attn cache
    ([2, NB, bs, H, D] storage viewed as [NB, 2, H, bs, D])."""
    h, bs, d, dtype = 8, 16, 128, torch.bfloat16
    lens = {"doc-a": 256, "doc-b": 512, "doc-c": 128}
    kv = {k: randn((2, h, n, d), dtype, 50 + i) for i, (k, n) in enumerate(lens.items())}
    owners = ["doc-b", "doc-a", "doc-c", "doc-b"]          # four 64-token target chunks
    starts = [300, 10, 64, 0]
    ids, dp, tp = [], [], []
    for c, (o, s) in enumerate(zip(owners, starts)):
        ids += [o] * 64
        dp += list(range(s, s + 64))
        tp += list(range(64 * c, 64 * c + 64))
    mapping = MultiDonorPositionMapping(tuple(ids), tuple(dp), tuple(tp))
    assert mapping.needs_correction
    storage = randn((2, 24, bs, h, d), dtype, 60)
    bt = torch.randperm(24, generator=gen(61))[:16].to(torch.int32)
    cache_dev = storage.to(dev).permute(1, 0, 3, 2, 4)
    composite_scatter_paged(cache_dev, {k: v.to(dev) for k, v in kv.items()}, bt.to(dev),
                            mapping, rope_base=1e4)
    want = storage.permute(1, 0, 3, 2, 4).clone()
    for did in lens:
        sub = mapping.for_donor(did)
        ref.rope_correct_scatter_paged(want, kv[did], bt, torch.tensor(sub.donor_positions),
                                       torch.tensor(sub.target_positions), rope_base=1e4)
    _check(cache_dev, want, True)


def test_composite_rejects_bad_inputs(dev):
    h, d, dtype = 2, 64, torch.bfloat16
    cache = [torch.zeros((8, 2, h, 16, d), dtype=dtype, device=dev)]
    donor = [[torch.zeros((2, h, 32, d), dtype=dtype, device=dev)]]
    idx = torch.zeros(4, dtype=torch.int32, device=dev)
    bt = torch.arange(8, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):   # donor with a wrong head count
        composite_scatter_paged_layers(
            cache, [[torch.zeros((2, h + 1, 32, d), dtype=dtype, device=dev)]], bt, idx, idx,
            idx)
    with pytest.raises(TypeError):    # dtype mismatch
        composite_scatter_paged_layers(
            cache, [[torch.zeros((2, h, 32, d), dtype=torch.float16, device=dev)]], bt, idx,
            idx, idx)
    with pytest.raises(ValueError):   # layer count mismatch
        composite_scatter_paged_layers(cache, [donor[0] * 2], bt, idx, idx, idx)
    with pytest.raises(ValueError):   # pair arrays of different lengths
        composite_scatter_paged_layers(cache, donor, bt, idx[:3], idx, idx)
    with pytest.raises(ValueError):   # duplicate targets in a mapping
        composite_scatter_paged(cache[0], [donor[0][0]], bt,
                                MultiDonorPositionMapping(("a", "a"), (0, 1), (3, 3)))


def test_composite_empty_inputs(dev):
    """No pairs, or pairs that all name no donor, leave the caches untouched."""
    h, d, dtype = 2, 64, torch.bfloat16
    base = [randn((8, 2, h, 16, d), dtype, 400 + l).to(dev) for l in range(2)]
    caches = [c.clone() for c in base]
    donors = [[randn((2, h, 32, d), dtype, 410 + l).to(dev) for l in range(2)]]
    bt = torch.arange(8, dtype=torch.int32, device=dev)
    empty = torch.zeros(0, dtype=torch.int32, device=dev)
    composite_scatter_paged_layers(caches, donors, bt, empty, empty, empty)
    bad = torch.tensor([1, 5, -1], dtype=torch.int32, device=dev)     # no such donors
    pos = torch.tensor([0, 1, 2], dtype=torch.int32, device=dev)
    composite_scatter_paged_layers(caches, donors, bt, bad, pos, pos)
    composite_scatter_paged(caches[0], [donors[0][0]], bt, MultiDonorPositionMapping())
    for a, b in zip(caches, base):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("rope", [True, False], ids=["rope", "copy"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n_donors", [3, 19])
def test_grouped_composite_matches_indexed(dev, dtype, rope, n_donors):
    """The donor-grouped launch (pairs grouped and padded by donor on the host, one launch per
    16 donors) lands the indexed launch's bits, skipped pairs included; 19 donors take two
    launches. Donors of different lengths, one a strided view, one a staged window whose row 0
    is a later sequence position."""
    layers, h, bs = 3, 4, 16
    d = 64 if dtype == torch.float32 else 128
    lens = [300 + 37 * k for k in range(n_donors)]
    firsts = [0] * n_donors
    firsts[-1] = 64
    donors = [[_donor(n, h, d, dtype, 100 * k + l, pad=40 if k == 1 else 0)
               for l in range(layers)] for k, n in enumerate(lens)]
    nb, nb_seq = 160, 128
    bt = torch.randperm(nb, generator=gen(15))[:nb_seq].to(torch.int32)
    didx, dpos, tpos = _plan(lens, nb_seq, bs, 64, 16 + n_donors, skip_frac=0.1)
    dpos = torch.where(didx == n_donors - 1, dpos + 64, dpos)  # the window's true positions
    base = _caches(layers, nb, h, bs, d, dtype, 17)
    dd = [[t.to(dev) for t in per] for per in donors]
    want = [c.to(dev) for c in base]
    composite_scatter_paged_layers(want, dd, bt.to(dev), didx, dpos, tpos, rope=rope,
                                   rope_base=5e5, donor_first_positions=firsts)
    got = [c.to(dev) for c in base]
    call = prepare_composite_scatter_paged_layers(got, dd, bt.to(dev), didx.to(dev), dpos, tpos,
                                                  rope=rope, rope_base=5e5,
                                                  donor_first_positions=firsts)
    assert len(call.launches) == (2 if n_donors > 16 else 1)
    call()
    for g_, w in zip(got, want):
        assert torch.equal(g_.view(torch.uint8), w.view(torch.uint8))
