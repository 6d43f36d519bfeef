"""GPU parity: batched (multi-request) entry points against the oracle, request by request.

Requests share one paged pool with their own (permuted, disjoint) block tables, as in a
serving batch; each request's result must match the oracle run on that request alone.
"""

from __future__ import annotations

import pytest
import torch

from oracle import ref_cpu as ref
from semblend_amd import triton_kernels as tk
from tests.helpers import assert_attn_close, gen, randn

pytestmark = pytest.mark.gpu


def _batch(ctx, nrows, hq, hkv, d, dtype, seed, bs=16):
    """Shared pool, per-request block tables (rows of a padded table), positions, queries."""
    g = gen(seed)
    nblk = [(c + bs - 1) // bs for c in ctx]
    pool = sum(nblk) + 7
    kv = randn((pool, 2, hkv, bs, d), dtype, seed + 1)
    perm = torch.randperm(pool, generator=g)
    tables = torch.full((len(ctx), max(nblk)), -1, dtype=torch.int32)
    at = 0
    for r, n in enumerate(nblk):
        tables[r, :n] = perm[at:at + n].to(torch.int32)
        at += n
    pos = [torch.randperm(c, generator=g)[:n].sort().values.to(torch.int32)
           for c, n in zip(ctx, nrows)]
    q = randn((sum(nrows), hq, d), dtype, seed + 2)
    return kv, tables, nblk, pos, q


def _check(kv, tables, nblk, pos, q, out, nrows):
    at = 0
    for r, n in enumerate(nrows):
        if n == 0:
            continue
        want = ref.partial_attention_paged(q[at:at + n], kv, tables[r, :nblk[r]], pos[r])
        assert_attn_close(out[at:at + n], want)
        at += n


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_varlen_llama_shape(dev, dtype):
    ctx, nrows = [512, 1024, 1536, 2048], [40, 100, 200, 300]
    kv, tables, nblk, pos, q = _batch(ctx, nrows, 32, 8, 128, dtype, 100)
    out = tk.partial_prefill_attention_paged_varlen(
        q.to(dev), kv.to(dev), tables.to(dev), torch.cat(pos).to(dev), nrows, nblk)
    _check(kv, tables, nblk, pos, q, out, nrows)


def test_varlen_matches_single_calls(dev):
    ctx, nrows = [2048, 700, 1300], [150, 60, 90]
    kv, tables, nblk, pos, q = _batch(ctx, nrows, 28, 4, 128, torch.bfloat16, 110)
    kvd, qd = kv.to(dev), q.to(dev)
    out = tk.partial_prefill_attention_paged_varlen(
        qd, kvd, tables.to(dev), torch.cat(pos).to(dev), nrows, nblk)
    at = 0
    for r, n in enumerate(nrows):
        single = tk.partial_prefill_attention_paged(qd[at:at + n], kvd,
                                                    tables[r, :nblk[r]].to(dev),
                                                    pos[r].to(dev))
        # same arithmetic up to the split of the key range (fp32 partial merges)
        assert float((out[at:at + n].float() - single.float()).abs().max()) <= 1e-2
        at += n


def test_varlen_empty_requests_and_many_launches(dev):
    # 20 requests (two launches of at most 16), two of them without rows
    ctx = [128 + 96 * i for i in range(20)]
    nrows = [0 if i in (3, 11) else 5 + 3 * i for i in range(20)]
    kv, tables, nblk, pos, q = _batch(ctx, nrows, 8, 2, 64, torch.bfloat16, 120)
    out = tk.partial_prefill_attention_paged_varlen(
        q.to(dev), kv.to(dev), tables.to(dev), torch.cat(pos).to(dev), nrows, nblk)
    _check(kv, tables, nblk, pos, q, out, nrows)


def test_varlen_fp32_per_request_path(dev):
    ctx, nrows = [300, 640], [20, 33]
    kv, tables, nblk, pos, q = _batch(ctx, nrows, 14, 2, 64, torch.float32, 130)
    out = tk.partial_prefill_attention_paged_varlen(
        q.to(dev), kv.to(dev), tables.to(dev), torch.cat(pos).to(dev), nrows, nblk)
    _check(kv, tables, nblk, pos, q, out, nrows)


def test_varlen_rejects_bad_plans(dev):
    kv, tables, nblk, pos, q = _batch([256, 256], [4, 4], 8, 2, 64, torch.bfloat16, 140)
    with pytest.raises(ValueError):
        tk.partial_prefill_attention_paged_varlen(
            q.to(dev), kv.to(dev), tables.to(dev), torch.cat(pos).to(dev), [4, 5], nblk)
    with pytest.raises(ValueError):
        tk.partial_prefill_attention_paged_varlen(
            q.to(dev), kv.to(dev), tables.to(dev), torch.cat(pos).to(dev), [4, 4],
            [nblk[0], tables.shape[1] + 1])


def test_kv_reuse_batch_llama_shape(dev):
    """A reduced Llama-3-8B batch (2 layers; contexts 1K..4K; 10-30% recompute): RoPE
    scatter of every request into the shared caches, then batched attention per layer, each
    checked against the oracle on that request alone."""
    import bench
    from semblend_amd.batch import KVReuseBatch
    from tests.helpers import assert_rope_close

    caches, reqs, theta = bench.llama_batch(dev, layers=2, ctx=(1024, 2048, 3072, 4096),
                                            pool_blocks=700, max_delta=1000, seed=7)
    before = [c.cpu() for c in caches]
    batch = KVReuseBatch(caches, reqs, rope_base=theta)
    batch.scatter_rope()
    for layer in range(2):
        want = before[layer].clone()
        for r in reqs:
            ref.rope_correct_scatter_paged(want, r.donor_kvs[layer].cpu(), r.block_table.cpu(),
                                           r.donor_positions.cpu(), r.target_positions.cpu(),
                                           rope_base=theta)
        got = caches[layer].cpu()
        assert torch.equal(got[:, 1].view(torch.int16), want[:, 1].view(torch.int16))
        assert_rope_close(got[:, 0], want[:, 0])
    # a repeated step reuses the prepared launches and lands the same bytes
    again = [c.clone() for c in caches]
    batch.scatter_rope()
    for a_, b_ in zip(caches, again):
        assert torch.equal(a_.view(torch.int16), b_.view(torch.int16))
    # rope=False copies like the plain multi-layer scatter, request by request
    got_plain = [c.to(dev) for c in before]
    KVReuseBatch(got_plain, reqs, rope_base=theta).scatter_rope(rope=False)
    want_plain = [c.to(dev) for c in before]
    for r in reqs:
        tk.scatter_donor_kv_paged_layers(want_plain, list(r.donor_kvs), r.block_table,
                                         r.donor_positions, r.target_positions)
    for a_, b_ in zip(got_plain, want_plain):
        assert torch.equal(a_.view(torch.int16), b_.view(torch.int16))
    q = randn((batch.num_rows, 32, 128), torch.bfloat16, 150).to(dev)
    for layer in range(2):
        out = batch.attention(layer, q)
        kv = caches[layer].cpu()
        for i, r in enumerate(reqs):
            a, b = batch.row_offsets[i], batch.row_offsets[i + 1]
            want = ref.partial_attention_paged(q[a:b].cpu(), kv, r.block_table.cpu(),
                                               r.compute_positions.cpu())
            assert_attn_close(out[a:b], want)
