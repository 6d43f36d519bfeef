"""The attention parity bar must accept a correct 16-bit computation and reject a plausible
wrong one, at the long contexts where outputs are small. CPU only.

A correct bf16 kernel is emulated on the CPU (fp32 scores scaled in fp32, P rounded to bf16
before the PV sum, output rounded once); the planted mistake is a split-key merge that
drops one of four key chunks, planted in a copy of the oracle's computation. The old
absolute-only bar (2e-2) accepts that mistake at these lengths; the per-row relative bar does
not.
"""

from __future__ import annotations

import math

import torch

from oracle import ref_cpu as ref
from tests.helpers import ATTN_16_ATOL, attn_row_violations, gen, randn


def _paged_case(ctx: int, rows: int, hq: int, hkv: int, d: int, seed: int):
    bs = 16
    nb = ctx // bs
    kv = randn((nb, 2, hkv, bs, d), torch.bfloat16, seed)
    bt = torch.randperm(nb, generator=gen(seed + 1)).to(torch.int32)
    pos = (ctx - 1 - torch.randperm(ctx // 4, generator=gen(seed + 2))[:rows]).sort().values
    q = randn((rows, hq, d), torch.bfloat16, seed + 3)
    return q, kv, bt, pos.to(torch.int32)


def _emulated_bf16(q, kv, bt, pos, drop_chunk: int | None = None, n_chunks: int = 4):
    """bf16 attention with the kernel's roundings; ``drop_chunk`` leaves out one of
    ``n_chunks`` equal key ranges of every row (a merge that lost a partial)."""
    rows, hq, d = q.shape
    hkv = kv.shape[2]
    group = hq // hkv
    k, v = ref.gather_paged_kv(kv, bt, int(pos.max()) + 1)
    k = k.repeat_interleave(group, dim=0)
    v = v.repeat_interleave(group, dim=0)
    qs = q.float() * (math.log2(math.e) / math.sqrt(d))
    out = torch.zeros((rows, hq, d))
    for r, p in enumerate(pos.tolist()):
        keys = torch.arange(p + 1)
        if drop_chunk is not None:
            span = (p + n_chunks) // n_chunks
            keys = keys[(keys // span) != drop_chunk]
        s = torch.einsum("hd,hkd->hk", qs[r], k[:, keys])
        pr = torch.exp2(s - s.amax(dim=1, keepdim=True)).to(torch.bfloat16).float()
        o = torch.einsum("hk,hkd->hd", pr, v[:, keys]) / pr.sum(dim=1, keepdim=True)
        out[r] = o
    return out.to(torch.bfloat16)


def test_row_bar_accepts_emulated_bf16_and_rejects_dropped_chunk():
    q, kv, bt, pos = _paged_case(ctx=65536, rows=8, hq=4, hkv=1, d=128, seed=40)
    want = ref.partial_attention_paged(q, kv, bt, pos)
    good = _emulated_bf16(q, kv, bt, pos)
    assert float((good.float() - want).abs().max()) <= ATTN_16_ATOL
    assert not bool(attn_row_violations(good, want).any())
    bad = _emulated_bf16(q, kv, bt, pos, drop_chunk=1)
    # the absolute bar alone cannot see it at this length ...
    assert float((bad.float() - want).abs().max()) <= ATTN_16_ATOL
    # ... the per-row bar rejects every row
    assert bool(attn_row_violations(bad, want).all())


def test_row_bar_margin_on_short_and_long_rows():
    """The emulated correct kernel stays well inside the per-row bar at both ends of the
    context (a single key, where the output is one V row, and thousands of keys)."""
    q, kv, bt, pos = _paged_case(ctx=4096, rows=8, hq=4, hkv=1, d=64, seed=50)
    pos = torch.cat([torch.tensor([0, 1, 2, 17], dtype=torch.int32), pos[4:]])
    want = ref.partial_attention_paged(q, kv, bt, pos)
    good = _emulated_bf16(q, kv, bt, pos).float()
    ratio = ((good - want).abs().amax(dim=-1) / want.abs().amax(dim=-1)).max()
    assert float(ratio) < 2.0 ** -7
