"""GPU parity on the engines' cache layouts: the vLLM flash-attn per-layer cache
[2, NB, bs, H, D] (synapse_kv_connector/model_runner_hook.py:461-463) and the TensorRT-LLM
cache [NB, 2, tpb, H, D] (semblend/integration/trtllm/kv_cache_adapter.py:1-12), next to the
standard [NB, 2, H, bs, D]. Every paged entry point addresses the cache through its strides,
so each layout is passed as its [NB, 2, H, bs, D] view (``rope_correction.standard_view``) and
the oracle runs on the same view of a CPU copy. Covered: plain and fused RoPE scatter (single
and multi-layer), the multi-layer permutations (delta and NoPE) that replace the per-layer
loop of model_runner_hook.py:519-585, and paged attention (single request and batched).
"""

from __future__ import annotations

import pytest
import torch

from oracle import ref_cpu as ref
from semblend_amd import rope_correction as rc
from semblend_amd import triton_kernels as tk
from tests.helpers import assert_attn_close, assert_bit_exact, assert_rope_close, gen, randn

pytestmark = pytest.mark.gpu

LAYOUTS = ["standard", "vllm", "trt"]


def _cache(layout, nb, h, bs, d, dtype, seed):
    """A cache in ``layout`` whose standard view holds N(0, 1) values (the axis orders of the
    three layouts are their own inverses)."""
    std = randn((nb, 2, h, bs, d), dtype, seed)
    return std.permute(*rc._LAYOUT_AXES[layout]).contiguous()


def _pairs(n_pos, n, seed, spread=300):
    g = gen(seed)
    tp = torch.randperm(n_pos, generator=g)[:n].to(torch.int32)
    dp = (tp.long() + torch.randint(-spread, spread, (n,), generator=g)).clamp(0, n_pos - 1)
    return dp.to(torch.int32), tp


@pytest.mark.parametrize("layout", LAYOUTS)
def test_scatter_layouts(dev, layout):
    nb, h, bs, d, s = 40, 4, 16, 128, 512
    cache = _cache(layout, nb, h, bs, d, torch.bfloat16, 1)
    donor = randn((2, h, s, d), torch.bfloat16, 2)
    bt = torch.randperm(nb, generator=gen(3))[:s // bs].to(torch.int32)
    dp, tp = _pairs(s, 300, 4)
    # plain scatter: the raw engine tensor must match bit for bit
    got = cache.to(dev)
    tk.scatter_donor_kv_paged(rc.standard_view(got, layout), donor.to(dev), bt.to(dev),
                              dp.to(dev), tp.to(dev))
    want = cache.clone()
    ref.scatter_donor_kv_paged(rc.standard_view(want, layout), donor, bt, dp, tp)
    assert_bit_exact(got, want)
    # fused RoPE scatter
    got = cache.to(dev)
    rc.rope_correct_scatter_paged(rc.standard_view(got, layout), donor.to(dev), bt.to(dev),
                                  dp.to(dev), tp.to(dev), rope_base=1e6)
    want = cache.clone()
    ref.rope_correct_scatter_paged(rc.standard_view(want, layout), donor, bt, dp, tp,
                                   rope_base=1e6)
    gv, wv = rc.standard_view(got.cpu(), layout), rc.standard_view(want, layout)
    assert_bit_exact(gv[:, 1], wv[:, 1])
    assert_rope_close(gv, wv)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("rope", [False, True])
def test_scatter_layers_layouts(dev, layout, rope):
    nb, h, bs, d, s, layers = 40, 4, 16, 128, 512, 3
    caches = [_cache(layout, nb, h, bs, d, torch.bfloat16, 10 + i) for i in range(layers)]
    donors = [randn((2, h, s, d), torch.bfloat16, 20 + i) for i in range(layers)]
    bt = torch.randperm(nb, generator=gen(5))[:s // bs].to(torch.int32)
    dp, tp = _pairs(s, 400, 6)
    got = [c.to(dev) for c in caches]
    views = [rc.standard_view(c, layout) for c in got]
    dd = [x.to(dev) for x in donors]
    if rope:
        rc.rope_correct_scatter_paged_layers(views, dd, bt.to(dev), dp.to(dev), tp.to(dev),
                                             rope_base=5e5)
    else:
        tk.scatter_donor_kv_paged_layers(views, dd, bt.to(dev), dp.to(dev), tp.to(dev))
    for layer in range(layers):
        want = caches[layer].clone()
        wv = rc.standard_view(want, layout)
        if rope:
            ref.rope_correct_scatter_paged(wv, donors[layer], bt, dp, tp, rope_base=5e5)
        else:
            ref.scatter_donor_kv_paged(wv, donors[layer], bt, dp, tp)
        gv = rc.standard_view(got[layer].cpu(), layout)
        assert_bit_exact(gv[:, 1], wv[:, 1])
        if rope:
            assert_rope_close(gv, wv)
        else:
            assert_bit_exact(got[layer], want)


def _permutation(seed):
    """Pairs with distinct targets that overlap the sources: shifted chunks, a swap and a
    three-cycle, so snapshot and sequential-copy semantics both matter."""
    g = gen(seed)
    src = torch.randperm(160, generator=g)[:100].tolist()
    tgt = torch.randperm(160, generator=g)[:100].tolist()
    perm = list(zip(src, tgt)) + [(3, 4), (4, 3), (7, 8), (8, 9), (9, 7)]
    return list({t: (s_, t) for s_, t in perm}.values())


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("nope", [False, True])
def test_permute_layers_layouts(dev, layout, nope):
    nb, h, bs, d, layers = 14, 4, 16, 128, 3
    caches = [_cache(layout, nb, h, bs, d, torch.bfloat16, 30 + i) for i in range(layers)]
    bt = torch.randperm(nb, generator=gen(7))[:10].to(torch.int32)
    perm = _permutation(8)
    got = [c.to(dev) for c in caches]
    fn = rc.nope_permute_paged_kv_layers if nope else rc.permute_paged_kv_with_rope_layers
    fn(got, bt.to(dev), perm, rope_base=1e6, layout=layout)
    oracle = ref.nope_permute_paged_kv if nope else ref.permute_paged_kv_with_rope
    for layer in range(layers):
        want = caches[layer].clone()
        oracle(rc.standard_view(want, layout), bt, perm, rope_base=1e6)
        gv = rc.standard_view(got[layer].cpu(), layout)
        wv = rc.standard_view(want, layout)
        assert_bit_exact(gv[:, 1], wv[:, 1])
        assert_rope_close(gv, wv)


@pytest.mark.parametrize("nope", [False, True])
def test_permute_layers_equals_single_layer_calls(dev, nope):
    """On the standard layout the multi-layer launch lands the same bytes as the drop-in
    single-layer function called once per layer; a prepared launch run twice equals two
    rounds of single-layer calls; layer groups (a small workspace cap) change nothing."""
    nb, h, bs, d, layers = 14, 2, 16, 64, 4
    caches = [randn((nb, 2, h, bs, d), torch.float16, 40 + i).to(dev) for i in range(layers)]
    bt = torch.randperm(nb, generator=gen(9))[:10].to(torch.int32).to(dev)
    perm = _permutation(11)
    single = rc.nope_permute_paged_kv if nope else rc.permute_paged_kv_with_rope
    want = [c.clone() for c in caches]
    for _ in range(2):
        for c in want:
            single(c, bt, perm, rope_base=1e4)
    got = [c.clone() for c in caches]
    call = rc.prepare_permute_paged_kv_layers(got, bt, perm, rope_base=1e4, nope=nope)
    call()
    call()
    grouped = [c.clone() for c in caches]
    # snapshot bytes per layer: K and V of every pair (delta), or K of every pair plus V of
    # every resolved move, one per distinct target (NoPE); the targets here are distinct
    per_layer = 2 * len(perm) * h * d * 2
    call = rc.prepare_permute_paged_kv_layers(grouped, bt, torch.tensor(perm), rope_base=1e4,
                                              nope=nope, max_workspace_bytes=2 * per_layer)
    assert len(call.launches) == 2
    call()
    call()
    for a, b, c in zip(got, want, grouped):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
        assert torch.equal(c.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("layout", LAYOUTS)
def test_paged_attention_layouts(dev, layout):
    nb, hkv, hq, bs, d, s = 80, 4, 28, 16, 128, 1024
    cache = _cache(layout, nb, hkv, bs, d, torch.bfloat16, 50)
    bt = torch.randperm(nb, generator=gen(51))[:s // bs].to(torch.int32)
    pos = torch.randperm(s, generator=gen(52))[:150].sort().values.to(torch.int32)
    q = randn((150, hq, d), torch.bfloat16, 53)
    kd = cache.to(dev)
    out = tk.partial_prefill_attention_paged(q.to(dev), rc.standard_view(kd, layout),
                                             bt.to(dev), pos.to(dev))
    want = ref.partial_attention_paged(q, rc.standard_view(cache, layout), bt, pos)
    assert_attn_close(out, want)
    # the same values in the standard layout give the same bits
    std = rc.standard_view(cache, layout).contiguous().to(dev)
    out_std = tk.partial_prefill_attention_paged(q.to(dev), std, bt.to(dev), pos.to(dev))
    assert torch.equal(out.view(torch.int16), out_std.view(torch.int16))
    # batched entry on the same cache, two requests
    tables = torch.full((2, s // bs), -1, dtype=torch.int32)
    tables[0] = bt
    tables[1, :32] = bt[:32]
    pos2 = torch.randperm(512, generator=gen(54))[:40].sort().values.to(torch.int32)
    q2 = randn((190, hq, d), torch.bfloat16, 55)
    outb = tk.partial_prefill_attention_paged_varlen(
        q2.to(dev), rc.standard_view(kd, layout), tables.to(dev),
        torch.cat([pos, pos2]).to(dev), [150, 40], [s // bs, 32])
    assert_attn_close(outb[:150], ref.partial_attention_paged(q2[:150], rc.standard_view(
        cache, layout), bt, pos))
    assert_attn_close(outb[150:], ref.partial_attention_paged(q2[150:], rc.standard_view(
        cache, layout), bt[:32], pos2))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_trt_64_token_blocks(dev, dtype):
    """TensorRT-LLM's common 64-token blocks [NB, 2, 64, H, D]: scatter bit-exact, the fused
    RoPE scatter within the RoPE bar, the multi-layer delta permutation and paged attention,
    each against the oracle on the standard view."""
    nb, h, bs, d, s = 24, 4, 64, 128, 1024
    cache = _cache("trt", nb, h, bs, d, dtype, 60)
    donor = randn((2, h, s, d), dtype, 61)
    bt = torch.randperm(nb, generator=gen(62))[:s // bs].to(torch.int32)
    dp, tp = _pairs(s, 700, 63)
    got = cache.to(dev)
    tk.scatter_donor_kv_paged(rc.standard_view(got, "trt"), donor.to(dev), bt.to(dev),
                              dp.to(dev), tp.to(dev))
    want = cache.clone()
    ref.scatter_donor_kv_paged(rc.standard_view(want, "trt"), donor, bt, dp, tp)
    assert_bit_exact(got, want)
    got = cache.to(dev)
    rc.rope_correct_scatter_paged(rc.standard_view(got, "trt"), donor.to(dev), bt.to(dev),
                                  dp.to(dev), tp.to(dev), rope_base=1e6)
    want = cache.clone()
    ref.rope_correct_scatter_paged(rc.standard_view(want, "trt"), donor, bt, dp, tp,
                                   rope_base=1e6)
    gv, wv = rc.standard_view(got.cpu(), "trt"), rc.standard_view(want, "trt")
    assert_bit_exact(gv[:, 1], wv[:, 1])
    assert_rope_close(gv, wv)
    # permutation over two layers
    caches = [_cache("trt", nb, h, bs, d, dtype, 64 + i) for i in range(2)]
    perm = [(a_, b_) for a_, b_ in zip(torch.randperm(s, generator=gen(66))[:300].tolist(),
                                      torch.randperm(s, generator=gen(67))[:300].tolist())]
    perm = list({t: (s_, t) for s_, t in perm}.values())
    got = [c.to(dev) for c in caches]
    rc.permute_paged_kv_with_rope_layers(got, bt.to(dev), perm, rope_base=1e6, layout="trt")
    for layer in range(2):
        want = caches[layer].clone()
        ref.permute_paged_kv_with_rope(rc.standard_view(want, "trt"), bt, perm, rope_base=1e6)
        gv = rc.standard_view(got[layer].cpu(), "trt")
        wv = rc.standard_view(want, "trt")
        assert_bit_exact(gv[:, 1], wv[:, 1])
        assert_rope_close(gv, wv)
    # attention over the 64-token-block cache
    pos = torch.randperm(s, generator=gen(68))[:120].sort().values.to(torch.int32)
    q = randn((120, 28, d), dtype, 69)
    out = tk.partial_prefill_attention_paged(q.to(dev), rc.standard_view(cache.to(dev), "trt"),
                                             bt.to(dev), pos.to(dev))
    assert_attn_close(out, ref.partial_attention_paged(q, rc.standard_view(cache, "trt"), bt,
                                                       pos))
