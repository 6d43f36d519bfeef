"""GPU: the no-allocation paged attention entry (sb_partial_attention_paged_noalloc), called
through the C ABI, gives bit-identical results to sb_partial_attention_paged (same kernels,
same plan, partials in the library's fixed array instead of a caller workspace) on two calls
in a row, the second smaller; a call whose partials exceed the array is refused before any
launch. Kept last in collection order: it leaves the array holding the last call's partials.
"""

from __future__ import annotations

import math

import pytest
import torch

from semblend_amd import _lib
from semblend_amd import triton_kernels as tk
from tests.helpers import gen, randn

pytestmark = pytest.mark.gpu


def _case(ctx, rows, hq, hkv, d, dtype, seed, bs=16):
    import bench

    g = gen(seed)
    nblk = ctx // bs
    pool = nblk + 5
    kv = randn((pool, 2, hkv, bs, d), dtype, seed + 1)
    bt = torch.randperm(pool, generator=g)[:nblk].to(torch.int32)
    pos = bench.recompute_positions(g, ctx, rows)
    q = randn((pos.numel(), hq, d), dtype, seed + 2)
    return q, kv, bt, pos


def _noalloc(q, kv, bt, pos, out):
    dev = q.device
    _, hq, d = q.shape
    nb, _, hkv, bs, _ = kv.shape
    with torch.cuda.device(dev):
        _lib.call("sb_partial_attention_paged_noalloc", out.data_ptr(), q.data_ptr(),
                  kv.data_ptr(), bt.data_ptr(), pos.data_ptr(), q.shape[0], hq, hkv, d, bs,
                  nb, bt.shape[0], 1.0 / math.sqrt(d), _lib.strides(q), _lib.strides(out),
                  _lib.strides(kv), _lib.dtype_code(q), _lib.stream_handle(dev))


def _need(q, kv, bt):
    _, hq, d = q.shape
    hkv, bs = kv.shape[2], kv.shape[3]
    return _lib.size_query("sb_partial_attention_paged_workspace_size", q.shape[0], hq, hkv, d,
                           bs, bt.shape[0], _lib.dtype_code(q))


def test_noalloc_matches_allocating_entry_on_two_calls(dev):
    cap = _lib.size_query("sb_partial_attention_paged_noalloc_max_scratch")
    cases = [
        # the Qwen2.5-7B 16K-context workload (2458 rows, 28q/4kv): 72 MB of partials
        _case(16384, 2458, 28, 4, 128, torch.bfloat16, 900),
        # then a smaller call in another dtype and shape, whose plan also splits
        _case(4096, 300, 32, 8, 64, torch.float16, 910),
    ]
    for q, kv, bt, pos in cases:
        need = _need(q, kv, bt)
        assert 0 < need <= cap
        qd, kvd, btd, posd = q.to(dev), kv.to(dev), bt.to(dev), pos.to(dev)
        want = tk.partial_prefill_attention_paged(qd, kvd, btd, posd)
        got = torch.full_like(want, float("nan"))
        _noalloc(qd, kvd, btd, posd, got)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_refuses_oversized_partials(dev):
    # Llama-3-8B shape, 32768-token context, 9830 rows: several hundred MB of partials
    q, kv, bt, pos = _case(32768, 9830, 32, 8, 128, torch.bfloat16, 920)
    assert _need(q, kv, bt) > _lib.size_query("sb_partial_attention_paged_noalloc_max_scratch")
    qd, kvd, btd, posd = q.to(dev), kv.to(dev), bt.to(dev), pos.to(dev)
    out = torch.zeros_like(qd)
    with pytest.raises(RuntimeError, match="holds at most"):
        _noalloc(qd, kvd, btd, posd, out)
    torch.cuda.synchronize()
    assert not bool(out.any())
