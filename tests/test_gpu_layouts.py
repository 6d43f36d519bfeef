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


# ---- in-place RoPE, one delta per position, over many layers ----

def _delta_entries(n_pos, n, seed, max_delta=2048):
    """(positions, deltas): n random positions with deltas in [-max_delta, max_delta], plus
    edge entries: a position listed three times with different deltas, one listed twice,
    negative positions (blocks counted from the end of the table), positions past the table
    and zero deltas (neither is processed)."""
    g = gen(seed)
    pos = torch.randint(0, n_pos, (n,), generator=g).tolist()
    dl = torch.randint(-max_delta, max_delta + 1, (n,), generator=g).tolist()
    pos += [pos[0], pos[0], pos[1], -3, -n_pos, n_pos + 5, n_pos, 11, 12]
    dl += [17, -900, 5, 33, -7, 100, 100, 0, 0]
    return pos, dl


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_deltas_layers_layouts(dev, layout, dtype):
    """One call over three layers equals the TRT-LLM hook's loop of one-position
    apply_rope_delta_inplace calls per (layer, pair) (semblend_provider.py:305-318), on the
    oracle: same count returned, V untouched, K within the RoPE bar for rows rotated several
    times."""
    nb, h, bs, d, layers = 40, 4, 16, 128, 3
    caches = [_cache(layout, nb, h, bs, d, dtype, 30 + i) for i in range(layers)]
    bt = torch.randperm(nb, generator=gen(33))[:32].to(torch.int32)
    pos, dl = _delta_entries(32 * bs, 300, 34)
    got = [c.to(dev) for c in caches]
    n = rc.apply_rope_deltas_inplace_layers(got, bt.to(dev), pos, dl, rope_base=5e5,
                                            layout=layout)
    want_n = 0
    for c in caches:
        v = rc.standard_view(c, layout)
        for p, dd in zip(pos, dl):
            want_n += ref.apply_rope_delta_inplace(v, bt, [p], dd, rope_base=5e5)
    assert n == want_n == layers * 305   # 300 random entries + 5 edge entries processed
    for g_, c in zip(got, caches):
        gv, wv = rc.standard_view(g_.cpu(), layout), rc.standard_view(c, layout)
        assert_bit_exact(gv[:, 1], wv[:, 1])
        assert_rope_close(gv, wv, composed=True)


def test_rope_deltas_layers_equals_per_delta_calls(dev):
    """The Qwen2.5-0.5B caller pattern (fp32, [128, 2, 2, 16, 64], a delta in [-64, 64] per
    token): one multi-layer call with per-token deltas lands the same bits as one
    apply_rope_delta_inplace call per distinct delta and layer (same rotation arithmetic)."""
    import bench

    inp = bench.qwen05b_pipeline_inputs(0)
    layers = [randn((128, 2, 2, 16, 64), torch.float32, 40 + i).to(dev) for i in range(2)]
    per_delta = [c.clone() for c in layers]
    bt = inp["block_table"].to(dev)
    dl = inp["deltas"]
    n = rc.apply_rope_deltas_inplace_layers(layers, bt, torch.arange(1024), dl, rope_base=1e6)
    m = 0
    for c in per_delta:
        for delta, ps in bench.delta_groups(dl):
            m += rc.apply_rope_delta_inplace(c, bt, ps, delta, rope_base=1e6)
    assert n == m == 2 * int((dl != 0).sum())
    for a, b in zip(layers, per_delta):
        assert_bit_exact(a, b)


def test_rope_deltas_layers_7b_shape(dev):
    """28 layers of the Qwen2.5-7B cache ([2048, 2, 4, 16, 128] bf16, vLLM layout), every one
    of 13926 reused positions rotated by its chunk's delta (constant per 256-token chunk in
    [-2048, 2048]): one launch; layers 0, 13 and 27 against the oracle's per-delta calls."""
    g = gen(50)
    bt = torch.randperm(2048, generator=g)[:1024].to(torch.int32)
    pos = torch.randperm(16384, generator=g)[:13926].sort().values
    chunk_delta = torch.randint(-2048, 2049, (64,), generator=g)
    dl = chunk_delta[pos // 256]
    caches = [_cache("vllm", 2048, 4, 16, 128, torch.bfloat16, 60 + i) for i in range(28)]
    got = [c.to(dev) for c in caches]
    n = rc.apply_rope_deltas_inplace_layers(got, bt.to(dev), pos, dl, rope_base=1e6)
    assert n == 28 * int((dl != 0).sum())
    for layer in (0, 13, 27):
        want = caches[layer].clone()
        for c in range(64):
            sel = (pos // 256 == c)
            ref.apply_rope_delta_inplace(want, bt, pos[sel].tolist(), int(chunk_delta[c]),
                                         rope_base=1e6)
        gv = rc.standard_view(got[layer].cpu(), "vllm")
        wv = rc.standard_view(want, "vllm")
        assert_bit_exact(gv[:, 1], wv[:, 1])
        assert_rope_close(gv, wv)
