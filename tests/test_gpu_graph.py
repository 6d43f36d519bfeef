"""GPU: the entry points captured in a HIP graph give the eager result on every replay.

Serving loops replay captured launch sequences; the library launches on torch's current
stream and allocates nothing itself, so capture works as long as nothing in a call needs the
host. Each graph is replayed several times with eager work and synchronisations in between,
and every replay is compared bit for bit with the eager result.
"""

from __future__ import annotations

import pytest
import torch

from semblend_amd import rope_correction as rc
from semblend_amd import triton_kernels as tk
from tests.helpers import gen, randn

pytestmark = pytest.mark.gpu


def _capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def _noise(dev):
    """Unrelated eager work between replays."""
    x = torch.randn(1 << 20, device=dev)
    return float((x * 2).sum())


def test_graph_attention_paged(dev):
    hq, hkv, d, bs, seq, rows = 28, 4, 128, 16, 4096, 300
    nb = seq // bs + 8
    kv = randn((nb, 2, hkv, bs, d), torch.bfloat16, 1).to(dev)
    bt = torch.randperm(nb, generator=gen(2))[: seq // bs].to(torch.int32).to(dev)
    pos = torch.randperm(seq, generator=gen(3))[:rows].sort().values.to(torch.int32).to(dev)
    q = randn((rows, hq, d), torch.bfloat16, 4).to(dev)
    out = torch.empty_like(q)
    tk.partial_prefill_attention_paged(q, kv, bt, pos, out=out)
    torch.cuda.synchronize()
    want = out.clone()
    g = _capture(lambda: tk.partial_prefill_attention_paged(q, kv, bt, pos, out=out))
    for _ in range(3):
        out.zero_()
        _noise(dev)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))


def test_graph_scatter_layers(dev):
    layers, hkv, d, bs, seq, pool = 4, 4, 128, 16, 2048, 160
    caches = [torch.zeros((pool, 2, hkv, bs, d), dtype=torch.bfloat16, device=dev)
              for _ in range(layers)]
    donors = [randn((2, hkv, seq, d), torch.bfloat16, 10 + i).to(dev) for i in range(layers)]
    bt = torch.randperm(pool, generator=gen(5))[: seq // bs].to(torch.int32).to(dev)
    dp = torch.randperm(seq, generator=gen(6))[:1500].to(torch.int32).to(dev)
    tp = torch.randperm(seq, generator=gen(7))[:1500].to(torch.int32).to(dev)
    tk.scatter_donor_kv_paged_layers(caches, donors, bt, dp, tp)
    torch.cuda.synchronize()
    want = [c.clone() for c in caches]
    g = _capture(lambda: tk.scatter_donor_kv_paged_layers(caches, donors, bt, dp, tp))
    for _ in range(3):
        for c in caches:
            c.zero_()
        _noise(dev)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for c, w in zip(caches, want):
            assert torch.equal(c.view(torch.int16), w.view(torch.int16))


def test_graph_rope_inplace(dev):
    layers, heads, seq, d = 4, 4, 2048, 128
    k0 = randn((layers, heads, seq, d), torch.bfloat16, 20).to(dev)
    dp = torch.arange(seq, dtype=torch.int32)
    deltas = torch.randint(-2048, 2049, (seq // 256,), generator=gen(21))
    tp = (dp + deltas[dp.long() // 256]).to(torch.int32)
    dp, tp = dp.to(dev), tp.to(dev)
    k = k0.clone()
    rc.rope_correct_k_inplace(k, dp, tp, head_dim=d, rope_base=1e6)
    torch.cuda.synchronize()
    want = k.clone()
    g = _capture(lambda: rc.rope_correct_k_inplace(k, dp, tp, head_dim=d, rope_base=1e6))
    for _ in range(3):
        k.copy_(k0)
        _noise(dev)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(k.view(torch.int16), want.view(torch.int16))


def test_graph_prepare_scatter_inside_capture(dev):
    """A multi-layer RoPE scatter prepared while the stream is capturing (no eager warm-up
    of this call): preparation reads nothing back from the device then (the load policy
    takes device positions as distinct), and every replay equals the eager launch."""
    L, nb, h, bs, d = 3, 48, 2, 16, 128
    caches0 = [randn((nb, 2, h, bs, d), torch.bfloat16, 40 + i).to(dev) for i in range(L)]
    donors = [randn((2, h, 512, d), torch.bfloat16, 50 + i).to(dev) for i in range(L)]
    bt = torch.randperm(nb, generator=gen(60))[:40].to(torch.int32).to(dev)
    tp = torch.arange(0, 600, dtype=torch.int32, device=dev)
    dp = (tp % 300 + 10).to(torch.int32)  # donor rows repeat
    rc.inv_freq_table(5e5, d, dev)  # the table exists before capture, as after any warm-up
    want = [c.clone() for c in caches0]
    rc.prepare_scatter_paged_layers(want, donors, bt, dp, tp, 5e5)()
    caches = [c.clone() for c in caches0]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call = rc.prepare_scatter_paged_layers(caches, donors, bt, dp, tp, 5e5)
        call()
    assert call.args[-1] == 0  # distinct assumed under capture
    for _ in range(3):
        for c, c0 in zip(caches, caches0):
            c.copy_(c0)
        _noise(dev)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for c, w in zip(caches, want):
            assert torch.equal(c.view(torch.int16), w.view(torch.int16))


@pytest.mark.parametrize("layout", ["standard", "vllm"])
def test_graph_apply_rope_delta_short_list(dev, layout):
    """apply_rope_delta_inplace with a short position list passes the positions inside the
    launch (no upload), so the call can be captured; every replay of the in-place rotation
    (from the same starting cache) equals the eager call."""
    nb, h, bs, d = 24, 2, 16, 64
    shape = (nb, 2, h, bs, d) if layout == "standard" else (2, nb, bs, h, d)
    kv0 = randn(shape, torch.bfloat16, 30).to(dev)
    bt = torch.randperm(nb, generator=gen(31))[:16].to(torch.int32).to(dev)
    pos = torch.randperm(256, generator=gen(32))[:40].tolist() + [7, 7, 200]
    kv = kv0.clone()
    rc.apply_rope_delta_inplace(kv, bt, pos, 37, rope_base=1e6)
    torch.cuda.synchronize()
    want = kv.clone()
    kv.copy_(kv0)
    g = _capture(lambda: rc.apply_rope_delta_inplace(kv, bt, pos, 37, rope_base=1e6))
    for _ in range(3):
        kv.copy_(kv0)
        _noise(dev)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(kv.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("nope", [False, True])
def test_graph_prepared_permute_layers(dev, nope):
    """The prepared multi-layer permutation (the RoPE hook's per-request call) replays the
    eager permutation of vLLM-layout caches; it is not idempotent, so each replay starts from
    the original caches."""
    layers, nb, hkv, bs, d = 3, 14, 4, 16, 128
    std = [randn((nb, 2, hkv, bs, d), torch.bfloat16, 30 + i) for i in range(layers)]
    c0 = [s.permute(*rc._LAYOUT_AXES["vllm"]).contiguous().to(dev) for s in std]
    caches = [c.clone() for c in c0]
    bt = torch.randperm(nb, generator=gen(31))[:10].to(torch.int32).to(dev)
    g0 = gen(32)
    src = torch.randperm(160, generator=g0)[:100].tolist()
    tgt = torch.randperm(160, generator=g0)[:100].tolist()
    perm = list({t: (s_, t) for s_, t in zip(src, tgt)}.values())
    call = rc.prepare_permute_paged_kv_layers(caches, bt, perm, rope_base=1e6, nope=nope,
                                              layout="vllm")
    call()
    torch.cuda.synchronize()
    want = [c.clone() for c in caches]
    for c, o in zip(caches, c0):
        c.copy_(o)
    g = _capture(call)
    for _ in range(3):
        for c, o in zip(caches, c0):
            c.copy_(o)
        _noise(dev)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for c, w in zip(caches, want):
            assert torch.equal(c.view(torch.int16), w.view(torch.int16))


def test_graph_rope_scatter_layers(dev):
    layers, hkv, d, bs, seq, pool = 4, 4, 128, 16, 2048, 160
    caches = [torch.zeros((pool, 2, hkv, bs, d), dtype=torch.bfloat16, device=dev)
              for _ in range(layers)]
    donors = [randn((2, hkv, seq, d), torch.bfloat16, 40 + i).to(dev) for i in range(layers)]
    bt = torch.randperm(pool, generator=gen(41))[: seq // bs].to(torch.int32).to(dev)
    dp = torch.randperm(seq, generator=gen(42))[:1500].to(torch.int32).to(dev)
    tp = torch.randperm(seq, generator=gen(43))[:1500].to(torch.int32).to(dev)

    def step():
        rc.rope_correct_scatter_paged_layers(caches, donors, bt, dp, tp, rope_base=5e5)

    step()
    torch.cuda.synchronize()
    want = [c.clone() for c in caches]
    g = _capture(step)
    for _ in range(3):
        for c in caches:
            c.zero_()
        _noise(dev)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for c, w in zip(caches, want):
            assert torch.equal(c.view(torch.int16), w.view(torch.int16))


@pytest.mark.parametrize("backend", ["fused", "library"])
def test_graph_projection_paged(dev, backend):
    """The compacted projection with its K/V write, both backends (the library one runs the
    hipBLASLt GEMM through torch inside the graph)."""
    rows, hidden, hq, hkv, d, bs, seq = 600, 1024, 8, 2, 128, 16, 2048
    nb = seq // bs + 4
    x = randn((seq, hidden), torch.bfloat16, 50).to(dev)
    w = (randn(((hq + 2 * hkv) * d, hidden), torch.bfloat16, 51) * 0.03).to(dev)
    b = randn(((hq + 2 * hkv) * d,), torch.bfloat16, 52).to(dev)
    pos = torch.randperm(seq, generator=gen(53))[:rows].sort().values.to(torch.int32).to(dev)
    bt = torch.randperm(nb, generator=gen(54))[: seq // bs].to(torch.int32).to(dev)
    kv = torch.zeros((nb, 2, hkv, bs, d), dtype=torch.bfloat16, device=dev)
    out = {}

    def step():
        out["q"] = tk.qkv_projection_paged(x, w, pos, kv, bt, num_heads=hq, num_kv_heads=hkv,
                                           head_dim=d, qkv_bias=b, rope_base=1e6,
                                           backend=backend)

    step()
    torch.cuda.synchronize()
    want_q, want_kv = out["q"].clone(), kv.clone()
    g = _capture(step)
    for _ in range(3):
        kv.zero_()
        out["q"].zero_()
        _noise(dev)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out["q"].view(torch.int16), want_q.view(torch.int16))
        assert torch.equal(kv.view(torch.int16), want_kv.view(torch.int16))


@pytest.mark.parametrize("n", [300, 2000])
def test_graph_delta_rope_uploaded_positions(dev, n):
    """apply_rope_delta_inplace with more distinct positions than travel in the launch (the
    list is uploaded from pinned memory) and the multi-layer per-position form: captured, the
    uploads' staging buffers are kept, so every replay rotates the same rows by the same
    deltas as an eager call on a shadow copy (each replay applies the rotations once more)."""
    nb, h, bs, d = 160, 4, 16, 128
    caches = [randn((nb, 2, h, bs, d), torch.bfloat16, 80 + i).to(dev) for i in range(3)]
    bt = torch.randperm(nb, generator=gen(83))[:128].to(torch.int32).to(dev)
    pos = torch.randperm(128 * bs, generator=gen(84))[:n].tolist()
    dl = torch.randint(-500, 501, (n,), generator=gen(85)).tolist()

    def step(cs):
        rc.apply_rope_delta_inplace(cs[0], bt, pos, 37, rope_base=1e4)
        rc.apply_rope_deltas_inplace_layers(cs, bt, pos, dl, rope_base=1e4)

    start = [c.clone() for c in caches]
    shadow = [c.clone() for c in caches]
    g = _capture(lambda: step(caches))       # its warm-up runs one eager step on caches
    for c, s in zip(caches, start):
        c.copy_(s)
    for _ in range(3):
        step(shadow)
        _noise(dev)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for c, s in zip(caches, shadow):
            assert torch.equal(c.view(torch.int16), s.view(torch.int16))
    assert not torch.equal(caches[1].view(torch.int16), start[1].view(torch.int16))


def test_graph_attention_paged_planned(dev):
    hq, hkv, d, bs, seq, rows = 28, 4, 128, 16, 8192, 900
    nb = seq // bs + 8
    kv = randn((nb, 2, hkv, bs, d), torch.bfloat16, 90).to(dev)
    bt = torch.randperm(nb, generator=gen(91))[: seq // bs].to(torch.int32).to(dev)
    pos_h = torch.randperm(seq, generator=gen(92))[:rows].sort().values.to(torch.int32)
    pos = pos_h.to(dev)
    q = randn((rows, hq, d), torch.bfloat16, 93).to(dev)
    plan = tk.plan_partial_attention_paged(pos_h, hq, hkv, d, bs, seq // bs, torch.bfloat16,
                                           dev)
    out = torch.empty_like(q)
    tk.partial_prefill_attention_paged(q, kv, bt, pos, out=out, plan=plan)
    torch.cuda.synchronize()
    want = out.clone()
    g = _capture(lambda: tk.partial_prefill_attention_paged(q, kv, bt, pos, out=out, plan=plan))
    for _ in range(3):
        out.zero_()
        _noise(dev)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
