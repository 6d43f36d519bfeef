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
