"""GPU parity: partial-prefill attention against the fp32 oracle.

bf16 / fp16 outputs must be within 2e-2 absolute of the fp32 reference; fp32 inputs within
the reference suite's own 1e-4 absolute / 1e-3 relative. Cases restate
synapse_kv_connector/tests/test_triton_kernels.py:396-493 and add GQA + paged cases up to the
Qwen2.5-7B shape (28 q heads / 4 KV heads, head_dim 128, 16384-token context).
"""

from __future__ import annotations

import math

import pytest
import torch

import bench
from oracle import ref_cpu as ref
from semblend_amd import triton_kernels as tk
from tests.helpers import assert_attn_close, gen, randn, recompute_set

pytestmark = pytest.mark.gpu


# ---- dense drop-in (triton_kernels.py:655-734) ----

def test_dense_all_compute_fp32(dev):
    q, k, v = (randn((2, 8, 16), torch.float32, s) for s in (1, 2, 3))
    mask = torch.ones(8, dtype=torch.bool)
    got = tk.partial_prefill_attention(q.to(dev), k.to(dev), v.to(dev), mask.to(dev),
                                       1.0 / math.sqrt(16))
    assert_attn_close(got, ref.partial_prefill_attention(q, k, v, mask, 1.0 / math.sqrt(16)))


def test_dense_reuse_rows_zero_and_full_context(dev):
    q, k, v = (randn((2, 8, 16), torch.float32, s) for s in (4, 5, 6))
    mask = torch.tensor([True, False, True, False, True, False, True, False])
    got = tk.partial_prefill_attention(q.to(dev), k.to(dev), v.to(dev), mask.to(dev)).cpu()
    for p in (1, 3, 5, 7):
        assert torch.all(got[:, p] == 0)
    assert_attn_close(got, ref.partial_prefill_attention(q, k, v, mask))
    q1, k1, v1 = (randn((1, 4, 8), torch.float32, s) for s in (7, 8, 9))
    m1 = torch.tensor([False, False, False, True])
    got1 = tk.partial_prefill_attention(q1.to(dev), k1.to(dev), v1.to(dev), m1.to(dev))
    assert_attn_close(got1, ref.partial_prefill_attention(q1, k1, v1, m1))


def test_dense_empty_mask(dev):
    q = randn((2, 4, 8), torch.float32, 10).to(dev)
    got = tk.partial_prefill_attention(q, q, q, torch.zeros(4, dtype=torch.bool, device=dev))
    assert torch.all(got == 0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("seq_len", [1, 77, 300, 1000])
def test_dense_mfma(dev, dtype, head_dim, seq_len):
    h = 3
    q, k, v = (randn((h, seq_len, head_dim), dtype, 20 + s) for s in range(3))
    mask = torch.rand(seq_len, generator=gen(seq_len)) < 0.3
    mask[-1] = True
    got = tk.partial_prefill_attention(q.to(dev), k.to(dev), v.to(dev), mask.to(dev))
    want = ref.partial_prefill_attention(q, k, v, mask)
    assert got.dtype == dtype
    assert torch.all(got.cpu()[:, ~mask] == 0)
    assert_attn_close(got, want)


@pytest.mark.parametrize("n_rows", [1, 40, 700])
def test_dense_split_from_device_row_count(dev, n_rows):
    """The dense drop-in knows its row count only on the device, so its kernels derive the
    key-range split from that count: a few rows of a long context run in many chunks (40
    rows of 8192 keys: 512-key chunks, merged by the general path past four chunks), more
    rows in fewer; the launch and the workspace cover every count."""
    h, s = 4, 8192
    q, k, v = (randn((h, s, 128), torch.bfloat16, 320 + i) for i in range(3))
    mask = torch.zeros(s, dtype=torch.bool)
    mask[torch.randperm(s, generator=gen(323 + n_rows))[:n_rows]] = True
    mask[s - 1] = True
    got = tk.partial_prefill_attention(q.to(dev), k.to(dev), v.to(dev), mask.to(dev))
    assert torch.all(got.cpu()[:, ~mask] == 0)
    assert_attn_close(got, ref.partial_prefill_attention(q, k, v, mask))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_dense_other_head_dim(dev, dtype):
    """head_dim 96 takes the general (non-MFMA) kernel."""
    q, k, v = (randn((2, 130, 96), dtype, 30 + s) for s in range(3))
    mask = torch.rand(130, generator=gen(31)) < 0.5
    got = tk.partial_prefill_attention(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.3)
    assert_attn_close(got, ref.partial_prefill_attention(q, k, v, mask, 0.3))


# ---- GQA over a paged cache ----

def _paged_case(hq, hkv, d, seq_len, n_rows, dtype, seed, nb=None, bs=16):
    nblk = (seq_len + bs - 1) // bs
    nb = nb or nblk + 7
    kv = randn((nb, 2, hkv, bs, d), dtype, seed)
    bt = torch.randperm(nb, generator=gen(seed + 1))[:nblk].to(torch.int32)
    pos = recompute_set(seq_len, n_rows, seed + 2, chunk=min(256, seq_len // 4 or 1))
    q = randn((pos.shape[0], hq, d), dtype, seed + 3)
    return q, kv, bt, pos


def test_paged_gqa_qwen05b_fp32(dev):
    """Qwen2.5-0.5B attention: 14 q heads / 2 KV heads, head_dim 64, fp32, 1024 tokens,
    154 query rows drawn without replacement."""
    kv = randn((128, 2, 2, 16, 64), torch.float32, 40)
    bt = torch.randperm(128, generator=gen(41))[:64].to(torch.int32)
    pos = torch.randperm(1024, generator=gen(42))[:154].sort().values.to(torch.int32)
    q = randn((154, 14, 64), torch.float32, 43)
    got = tk.partial_prefill_attention_paged(q.to(dev), kv.to(dev), bt.to(dev), pos.to(dev))
    assert_attn_close(got, ref.partial_attention_paged(q, kv, bt, pos))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv,d", [(28, 4, 128), (32, 8, 128), (14, 2, 64), (8, 8, 128)])
def test_paged_gqa_mfma(dev, dtype, hq, hkv, d):
    q, kv, bt, pos = _paged_case(hq, hkv, d, 2048, 300, dtype, 50)
    got = tk.partial_prefill_attention_paged(q.to(dev), kv.to(dev), bt.to(dev), pos.to(dev))
    assert_attn_close(got, ref.partial_attention_paged(q, kv, bt, pos))


@pytest.mark.parametrize("bs", [24, 32, 1])
def test_paged_gqa_block_sizes(dev, bs):
    """Block sizes other than 16. 24 is not a power of two, so the block of a key is found
    by division and its offset with 64-bit products; 1 puts every key in its own block."""
    q, kv, bt, pos = _paged_case(28, 4, 128, 1500, 200, torch.bfloat16, 80 + bs, bs=bs)
    got = tk.partial_prefill_attention_paged(q.to(dev), kv.to(dev), bt.to(dev), pos.to(dev))
    assert_attn_close(got, ref.partial_attention_paged(q, kv, bt, pos))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("seq_len", [384, 383])
def test_paged_gqa_every_tile_count(dev, dtype, seq_len):
    """Every position of a short context is a query row, so the row tiles' key ranges grow
    from one 64-key tile to six (and, at 383, end one key short of a tile): the tile loop
    runs its two-tile body zero to two times and finishes with one or two tiles, for every
    combination."""
    q, kv, bt, _ = _paged_case(28, 4, 128, seq_len, 8, dtype, 70 + seq_len)
    pos = torch.arange(seq_len, dtype=torch.int32)
    q = randn((seq_len, 28, 128), dtype, 71 + seq_len)
    got = tk.partial_prefill_attention_paged(q.to(dev), kv.to(dev), bt.to(dev), pos.to(dev))
    assert_attn_close(got, ref.partial_attention_paged(q, kv, bt, pos))


def test_paged_gqa_position_major_layout(dev):
    """A cache stored [blocks, block_size, 2, kv_heads, head_dim] and viewed as
    [blocks, 2, kv_heads, block_size, head_dim]: the position stride (2·H·D) exceeds the
    head stride, and K and V of a position sit next to each other."""
    q, kv, bt, pos = _paged_case(32, 8, 128, 1200, 150, torch.bfloat16, 90)
    store = kv.permute(0, 3, 1, 2, 4).contiguous()        # [nb, bs, 2, H, D]
    view = store.to(dev).permute(0, 2, 3, 1, 4)           # [nb, 2, H, bs, D]
    assert not view.is_contiguous()
    got = tk.partial_prefill_attention_paged(q.to(dev), view, bt.to(dev), pos.to(dev))
    assert_attn_close(got, ref.partial_attention_paged(q, kv, bt, pos))


def test_paged_gqa_no_rows(dev):
    q, kv, bt, _ = _paged_case(28, 4, 128, 256, 8, torch.bfloat16, 95)
    got = tk.partial_prefill_attention_paged(q[:0].to(dev), kv.to(dev), bt.to(dev),
                                             torch.zeros(0, dtype=torch.int32, device=dev))
    assert got.shape == (0, 28, 128)


def test_paged_gqa_long_context_many_chunks(dev):
    """A 65536-token context with few rows: the planner splits the key range into 512-key
    chunks to fill the GPU, so the last rows span 128 chunks that the merge combines. Rows
    at the start, at chunk limits and at the last position, plus random ones."""
    ctx, bs = 65536, 16
    nblk = ctx // bs
    kv = randn((nblk + 3, 2, 1, bs, 128), torch.bfloat16, 96)
    bt = torch.randperm(nblk + 3, generator=gen(97))[:nblk].to(torch.int32)
    pos = torch.cat([torch.tensor([0, 1, 16383, 16384, 32767, 49152, 65534, 65535]),
                     torch.randint(0, ctx, (40,), generator=gen(98))]).unique()
    pos = pos.sort().values.to(torch.int32)
    q = randn((pos.shape[0], 8, 128), torch.bfloat16, 99)
    got = tk.partial_prefill_attention_paged(q.to(dev), kv.to(dev), bt.to(dev), pos.to(dev))
    assert_attn_close(got, ref.partial_attention_paged(q, kv, bt, pos))


def test_paged_gqa_unsorted_positions(dev):
    q, kv, bt, pos = _paged_case(28, 4, 128, 1024, 200, torch.bfloat16, 60)
    perm = torch.randperm(pos.shape[0], generator=gen(61))
    q, pos = q[perm].contiguous(), pos[perm].contiguous()
    got = tk.partial_prefill_attention_paged(q.to(dev), kv.to(dev), bt.to(dev), pos.to(dev))
    assert_attn_close(got, ref.partial_attention_paged(q, kv, bt, pos))


def test_paged_gqa_full_size_7b(dev):
    """The 7B attention workload at full size: 16384-token context, 2458 query rows
    (first 256 tokens, two random 256-token chunks, the rest scattered), 28/4 heads, bf16.
    Every output row is compared with the oracle."""
    q, kv, bt, pos = _paged_case(28, 4, 128, 16384, 2458, torch.bfloat16, 70, nb=2048)
    assert pos.shape[0] == 2458
    got = tk.partial_prefill_attention_paged(q.to(dev), kv.to(dev), bt.to(dev), pos.to(dev))
    want = ref.partial_attention_paged(q, kv, bt, pos)
    assert_attn_close(got.cpu(), want)


def test_paged_gqa_bench_workload(dev):
    """The attention phase that bench.py times, on its own inputs (built by the same seeded
    code on the device): all 2458 rows of all 28 q-heads against the oracle."""
    inp = bench.build_inputs(dev)
    q, kv, pos = inp["attn_q"], inp["attn_kv"], inp["attn_pos"]
    bt = inp["block_table"]
    got = tk.partial_prefill_attention_paged(q, kv, bt, pos)
    want = ref.partial_attention_paged(q.cpu(), kv.cpu(), bt.cpu(), pos.cpu())
    assert_attn_close(got.cpu(), want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_paged_gqa_rising_scores_rescale(dev, dtype):
    """Scores that keep rising along the context, so the kernel's reference max must move
    (O and l rescaled, the next tile's scores shifted) many times within one row: K rows are
    scaled from 1 to 24 (bf16) or 1 to 4 (fp16) along the positions, so a late tile's
    scores exceed the first tile's maximum by far more than the 2^64 (bf16) or 2^8 (fp16)
    tile-sum bound of P. Rows at every 64-key tile boundary and at the end of the context,
    with several key chunks for the long rows."""
    hq, hkv, d, bs, ctx = 8, 2, 128, 16, 4096
    nb = ctx // bs
    top = 24.0 if dtype == torch.bfloat16 else 4.0
    kv = randn((nb, 2, hkv, bs, d), torch.float32, 120)
    scale = torch.linspace(1.0, top, ctx).view(nb, bs)          # per position
    kv[:, 0] *= scale[:, None, :, None]
    kv = kv.to(dtype)
    bt = torch.arange(nb, dtype=torch.int32)
    pos = torch.cat([torch.arange(63, ctx, 256), torch.tensor([0, 64, 4094, 4095]),
                     torch.randint(0, ctx, (60,), generator=gen(121))]).unique()
    pos = pos.sort().values.to(torch.int32)
    q = randn((pos.shape[0], hq, d), dtype, 122)
    got = tk.partial_prefill_attention_paged(q.to(dev), kv.to(dev), bt.to(dev), pos.to(dev))
    want = ref.partial_attention_paged(q, kv, bt, pos)
    # the softmax is peaked: most rows put nearly all weight on a few late keys
    assert float(want.abs().amax()) > 1.0
    assert_attn_close(got, want)


# ---- host-planned launches (split + longest-first order) ----

def test_paged_gqa_planned_bench_workload(dev):
    """The planned launch on the bench's 7B inputs: every row against the oracle, and a
    plan of other positions (same shape) is still correct, only slower."""
    inp = bench.build_inputs(dev)
    q, kv, pos, bt = inp["attn_q"], inp["attn_kv"], inp["attn_pos"], inp["block_table"]
    plan = tk.plan_partial_attention_paged(inp["pos_cpu"], 28, 4, 128, 16, bt.shape[0],
                                           torch.bfloat16, dev)
    assert plan.max_chunks >= 2 and plan.ks_rest < plan.ks_first
    got = tk.partial_prefill_attention_paged(q, kv, bt, pos, plan=plan)
    want = ref.partial_attention_paged(q.cpu(), kv.cpu(), bt.cpu(), pos.cpu())
    assert_attn_close(got.cpu(), want)
    other = recompute_set(16384, pos.shape[0], 5)
    plan2 = tk.plan_partial_attention_paged(other, 28, 4, 128, 16, bt.shape[0], torch.bfloat16,
                                            dev)
    got2 = tk.partial_prefill_attention_paged(q, kv, bt, pos, plan=plan2)
    assert_attn_close(got2.cpu(), want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv,d,seq,rows,bs", [(28, 4, 128, 4096, 600, 16),
                                                   (32, 8, 128, 8192, 800, 16),
                                                   (14, 2, 64, 3000, 450, 32),
                                                   (8, 8, 128, 2048, 300, 24)])
def test_paged_gqa_planned_shapes(dev, dtype, hq, hkv, d, seq, rows, bs):
    q, kv, bt, pos = _paged_case(hq, hkv, d, seq, rows, dtype, 130 + hq + bs, bs=bs)
    plan = tk.plan_partial_attention_paged(pos, hq, hkv, d, bs, bt.shape[0], dtype, dev)
    got = tk.partial_prefill_attention_paged(q.to(dev), kv.to(dev), bt.to(dev), pos.to(dev),
                                             plan=plan)
    assert_attn_close(got, ref.partial_attention_paged(q, kv, bt, pos))


def test_paged_gqa_planned_unsorted_and_fp32(dev):
    """Positions in any order (the plan reads them as given); fp32 takes the VALU kernel,
    for which the plan is empty."""
    q, kv, bt, pos = _paged_case(28, 4, 128, 2048, 400, torch.bfloat16, 140)
    perm = torch.randperm(pos.shape[0], generator=gen(141))
    q, pos = q[perm].contiguous(), pos[perm].contiguous()
    plan = tk.plan_partial_attention_paged(pos, 28, 4, 128, 16, bt.shape[0], torch.bfloat16, dev)
    got = tk.partial_prefill_attention_paged(q.to(dev), kv.to(dev), bt.to(dev), pos.to(dev),
                                             plan=plan)
    assert_attn_close(got, ref.partial_attention_paged(q, kv, bt, pos))
    q32, kv32 = q.float(), kv.float()
    plan32 = tk.plan_partial_attention_paged(pos, 28, 4, 128, 16, bt.shape[0], torch.float32,
                                             dev)
    assert plan32.max_chunks == 0 and plan32.order.numel() == 0
    got32 = tk.partial_prefill_attention_paged(q32.to(dev), kv32.to(dev), bt.to(dev),
                                               pos.to(dev), plan=plan32)
    assert_attn_close(got32, ref.partial_attention_paged(q32, kv32, bt, pos))
    with pytest.raises(ValueError, match="another shape"):
        tk.partial_prefill_attention_paged(q.to(dev)[:10], kv.to(dev), bt.to(dev),
                                           pos.to(dev)[:10], plan=plan)
