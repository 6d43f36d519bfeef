"""CPU oracle for SemBlend's KV-reuse path — TEST INFRASTRUCTURE ONLY.

This module restates, on CPU tensors, the reference's own CPU semantics for every function on
the path. The HIP kernels are compared against it in the tests, and it is the CPU baseline that
``bench.py`` times. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
cpu_baseline leg may import it; the ``semblend_amd`` package never does.

Conventions (all cited reference paths are relative to the reference repository root):

* Floating-point work uses torch on the CPU, as the reference's fallbacks do, so inv_freq,
  angle products and rounding to the cache dtype are the reference's bit for bit; cos/sin
  are torch-CPU's.
* Bounds: pairs whose donor position, logical block or physical block is out of range are
  skipped, following the reference's GPU kernels (semblend_core/triton_kernels.py:106-108,
  :246-260; semblend_core/rope_correction.py:117-129). The reference's CPU fallbacks raise
  on such pairs instead; for in-range inputs both rules agree.
* Attention is evaluated in fp32 whatever the input dtype (an fp32 reference); for fp32
  inputs this is the reference's CPU computation exactly (triton_kernels.py:717-732).

Pinning (tests/test_oracle_*.py): every function is checked against the reference test
suite's own cases restated (synapse_kv_connector/tests/test_triton_kernels.py,
test_rope_correction.py, test_partial_attention.py), against float64 closed forms
(tests/golden/*.npz, written by tests/golden/make_golden.py from numpy, independently of this
module), against invariants (rotation group law, norm preservation, V untouched, reversibility)
and against planted mistakes that those checks must catch (tests/test_oracle_mutations.py).
"""

from __future__ import annotations

import math

import torch

__all__ = [
    "apply_rope_delta_inplace",
    "composite_scatter_paged",
    "gather_paged_kv",
    "inv_freq",
    "masked_qkv_projection",
    "nope_permute_paged_kv",
    "partial_attention_paged",
    "partial_prefill",
    "partial_prefill_attention",
    "permute_paged_kv_with_rope",
    "qkv_project_paged",
    "rope_correct_k",
    "rope_correct_scatter_paged",
    "rotate_interleaved",
    "scatter_donor_kv",
    "scatter_donor_kv_paged",
]


def inv_freq(rope_base: float, head_dim: int) -> torch.Tensor:
    """fp32 ``1 / base ** (arange(0, D, 2) / D)`` (semblend_core/rope_correction.py:234-238)."""
    return 1.0 / (rope_base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))


def rotate_interleaved(k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Interleaved rotation of the last dim in fp32 (semblend_core/rope_correction.py:317-326):
    ``even' = even*cos - odd*sin``, ``odd' = even*sin + odd*cos``."""
    k = k.float()
    even = k[..., 0::2]
    odd = k[..., 1::2]
    out = torch.zeros_like(k)
    out[..., 0::2] = even * cos - odd * sin
    out[..., 1::2] = even * sin + odd * cos
    return out


# ------------------------------------------------------------------------------------------
# Scatter
# ------------------------------------------------------------------------------------------

def scatter_donor_kv(target, donor, donor_positions, target_positions):
    """In place ``target[:, :, :, t] = donor[:, :, :, d]`` (triton_kernels.py:185-189), pairs
    outside either sequence skipped (:106-108)."""
    d = donor_positions.long()
    t = target_positions.long()
    keep = (d >= 0) & (d < donor.shape[3]) & (t >= 0) & (t < target.shape[3])
    d, t = d[keep], t[keep]
    if d.numel():
        target[:, :, :, t, :] = donor[:, :, :, d, :]
    return target


def _paged_slot(block_table, pos: int, block_size: int, num_blocks_total: int):
    """(physical block, offset) of a logical position, or None when out of range."""
    if pos < 0:
        return None
    lb = pos // block_size
    if lb >= block_table.shape[0]:
        return None
    pb = int(block_table[lb])
    if pb < 0 or pb >= num_blocks_total:
        return None
    return pb, pos % block_size


def scatter_donor_kv_paged(kv_cache, donor_kv, block_table, donor_positions, target_positions):
    """Per-pair loop of triton_kernels.py:338-354 with the donor-length check of :246-248."""
    num_blocks_total, _, _, block_size, _ = kv_cache.shape
    donor_len = donor_kv.shape[2]
    for i in range(donor_positions.shape[0]):
        d = int(donor_positions[i])
        t = int(target_positions[i])
        if d < 0 or d >= donor_len:
            continue
        slot = _paged_slot(block_table, t, block_size, num_blocks_total)
        if slot is None:
            continue
        kv_cache[slot[0], :, :, slot[1], :] = donor_kv[:, :, d, :]
    return kv_cache


# ------------------------------------------------------------------------------------------
# RoPE
# ------------------------------------------------------------------------------------------

def rope_correct_scatter_paged(kv_cache, donor_kv, block_table, donor_positions,
                               target_positions, rope_base=10000.0, head_dim=None):
    """Per-pair loop of rope_correction.py:296-328 (V copied, K rotated by t - d, rounded once
    to the cache dtype), with the kernel's bounds skips (:117-129)."""
    num_blocks_total, _, _, block_size, hd = kv_cache.shape
    head_dim = hd if head_dim is None else head_dim
    freq = inv_freq(rope_base, head_dim)
    donor_len = donor_kv.shape[2]
    for i in range(donor_positions.shape[0]):
        d = int(donor_positions[i])
        t = int(target_positions[i])
        if d < 0 or d >= donor_len:
            continue
        slot = _paged_slot(block_table, t, block_size, num_blocks_total)
        if slot is None:
            continue
        pb, off = slot
        theta = float(t - d) * freq
        kv_cache[pb, 1, :, off, :] = donor_kv[1, :, d, :]
        k = rotate_interleaved(donor_kv[0, :, d, :], torch.cos(theta), torch.sin(theta))
        kv_cache[pb, 0, :, off, :] = k.to(kv_cache.dtype)
    return kv_cache


def composite_scatter_paged(kv_cache, donor_kvs, block_table, donor_index, donor_positions,
                            target_positions, rope=True, rope_base=10000.0):
    """Multi-donor scatter as the reference composes it: the pairs are split by donor
    (``MultiDonorPositionMapping.for_donor``, semblend_core/multi_donor_types.py:70-78) and
    each donor's subset goes through the single-donor path, RoPE-corrected
    (rope_correction.py:296-328) or a plain copy (triton_kernels.py:338-354), donor by donor
    in index order. Pairs naming no donor in range are skipped."""
    donor_index = torch.as_tensor(donor_index)
    donor_positions = torch.as_tensor(donor_positions)
    target_positions = torch.as_tensor(target_positions)
    for k, donor_kv in enumerate(donor_kvs):
        sel = donor_index == k
        if not bool(sel.any()):
            continue
        if rope:
            rope_correct_scatter_paged(kv_cache, donor_kv, block_table, donor_positions[sel],
                                       target_positions[sel], rope_base=rope_base)
        else:
            scatter_donor_kv_paged(kv_cache, donor_kv, block_table, donor_positions[sel],
                                   target_positions[sel])
    return kv_cache


def rope_correct_k(k_tensor, donor_positions, target_positions, head_dim=128,
                   rope_base=10000.0):
    """rope_correction.py:362-399: clone, then for each pair in order rotate the row at the
    donor position by (t - d), rounding to the tensor dtype after each pair."""
    freq = inv_freq(rope_base, head_dim)
    deltas = (target_positions - donor_positions).float()
    theta = deltas.unsqueeze(-1) * freq.unsqueeze(0)
    cos_all, sin_all = torch.cos(theta), torch.sin(theta)
    result = k_tensor.clone()
    seq_len = k_tensor.shape[-2]
    for i in range(donor_positions.shape[0]):
        d = int(donor_positions[i])
        if d < 0 or d >= seq_len:
            continue
        row = result[..., d, :]
        result[..., d, :] = rotate_interleaved(row, cos_all[i], sin_all[i]).to(k_tensor.dtype)
    return result


def permute_paged_kv_with_rope(kv_cache, block_table, permutation, rope_base=10000.0):
    """rope_correction.py:427-476: snapshot every source (K and V), then write V copies and
    K rotated by (tgt - src) at the targets."""
    if not permutation:
        return
    num_blocks_total, _, _, block_size, head_dim = kv_cache.shape
    pairs = []
    for s, t in permutation:
        if _paged_slot(block_table, s, block_size, num_blocks_total) is None:
            continue
        if _paged_slot(block_table, t, block_size, num_blocks_total) is None:
            continue
        pairs.append((s, t))
    if not pairs:
        return
    src = torch.tensor([p[0] for p in pairs], dtype=torch.long)
    tgt = torch.tensor([p[1] for p in pairs], dtype=torch.long)
    sb = block_table[src // block_size].long()
    so = src % block_size
    src_k = kv_cache[sb, 0, :, so, :].clone()
    src_v = kv_cache[sb, 1, :, so, :].clone()
    tb = block_table[tgt // block_size].long()
    to = tgt % block_size
    kv_cache[tb, 1, :, to, :] = src_v
    freq = inv_freq(rope_base, head_dim)
    theta = (tgt - src).float().unsqueeze(-1) * freq.unsqueeze(0)
    k = rotate_interleaved(src_k, torch.cos(theta).unsqueeze(1), torch.sin(theta).unsqueeze(1))
    kv_cache[tb, 0, :, to, :] = k.to(kv_cache.dtype)


def nope_permute_paged_kv(kv_cache, block_table, permutation, rope_base=10000.0):
    """rope_correction.py:620-697 with its CPU path :786-823: K of every source snapshotted,
    V copied pair by pair IN ORDER (a later pair sees earlier copies), then
    K[tgt] = R(tgt) R(-src) K_snapshot in fp32, rounded once."""
    if not permutation:
        return
    num_blocks_total, _, _, block_size, head_dim = kv_cache.shape
    freq = inv_freq(rope_base, head_dim)
    snaps = []
    for s, t in permutation:
        s_slot = _paged_slot(block_table, s, block_size, num_blocks_total)
        t_slot = _paged_slot(block_table, t, block_size, num_blocks_total)
        if s_slot is None or t_slot is None:
            continue
        snaps.append((s, t, s_slot, t_slot, kv_cache[s_slot[0], 0, :, s_slot[1], :].clone()))
        kv_cache[t_slot[0], 1, :, t_slot[1], :] = kv_cache[s_slot[0], 1, :, s_slot[1], :]
    for s, t, _, t_slot, k in snaps:
        kf = k.float()
        ts, tt = float(s) * freq, float(t) * freq
        cs, ss, ct, st = torch.cos(ts), torch.sin(ts), torch.cos(tt), torch.sin(tt)
        even, odd = kf[:, 0::2], kf[:, 1::2]
        raw_even = even * cs + odd * ss
        raw_odd = -even * ss + odd * cs
        out = torch.zeros_like(kf)
        out[:, 0::2] = raw_even * ct - raw_odd * st
        out[:, 1::2] = raw_even * st + raw_odd * ct
        kv_cache[t_slot[0], 0, :, t_slot[1], :] = out.to(kv_cache.dtype)


def apply_rope_delta_inplace(kv_cache, block_table, positions, delta, rope_base=10000.0):
    """rope_correction.py:732-783: layout detection, one rotation per listed position
    (positions past the table skipped), count of positions processed returned."""
    if delta == 0 or not positions:
        return 0
    is_vllm = kv_cache.shape[0] == 2 and (kv_cache.ndim == 5 and kv_cache.shape[1] != 2)
    head_dim = kv_cache.shape[4]
    block_size = kv_cache.shape[2] if is_vllm else kv_cache.shape[3]
    freq = inv_freq(rope_base, head_dim)
    theta = float(delta) * freq
    cos_v, sin_v = torch.cos(theta), torch.sin(theta)
    modified = 0
    for pos in positions:
        blk_idx = pos // block_size
        if blk_idx >= block_table.shape[0]:
            continue
        blk = int(block_table[blk_idx])
        off = pos % block_size
        if is_vllm:
            kv_cache[0, blk, off, :, :] = rotate_interleaved(
                kv_cache[0, blk, off, :, :], cos_v, sin_v).to(kv_cache.dtype)
        else:
            kv_cache[blk, 0, :, off, :] = rotate_interleaved(
                kv_cache[blk, 0, :, off, :], cos_v, sin_v).to(kv_cache.dtype)
        modified += 1
    return modified


# ------------------------------------------------------------------------------------------
# Attention
# ------------------------------------------------------------------------------------------

def partial_prefill_attention(query, key, value, compute_mask, scale=None):
    """triton_kernels.py:717-732 evaluated in fp32: for each compute row i,
    softmax(scale * q_i K[:i+1]^T) V[:i+1]; other rows 0. Returns fp32 [H, S, D]."""
    num_heads, seq_len, head_dim = query.shape
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    q, k, v = query.float(), key.float(), value.float()
    out = torch.zeros((num_heads, seq_len, head_dim), dtype=torch.float32)
    for pos in torch.where(compute_mask.bool())[0].tolist():
        scores = torch.matmul(q[:, pos:pos + 1, :], k[:, :pos + 1, :].transpose(-2, -1)) * scale
        out[:, pos:pos + 1, :] = torch.matmul(torch.softmax(scores, dim=-1), v[:, :pos + 1, :])
    return out


def gather_paged_kv(kv_cache, block_table, num_tokens):
    """Dense fp32 K, V [Hkv, num_tokens, D] read from a paged [NB, 2, Hkv, bs, D] cache."""
    block_size = kv_cache.shape[3]
    t = torch.arange(num_tokens)
    pb = block_table[t // block_size].long()
    off = t % block_size
    k = kv_cache[pb, 0, :, off, :].permute(1, 0, 2).float()
    v = kv_cache[pb, 1, :, off, :].permute(1, 0, 2).float()
    return k, v


def partial_attention_paged(query, kv_cache, block_table, positions, scale=None):
    """GQA partial attention over a paged cache, in fp32: K/V gathered from the cache, KV
    heads repeated for their query-head group (query head h reads KV head h // group), then
    the per-row computation of triton_kernels.py:717-732. query [R, Hq, D] -> fp32 [R, Hq, D]."""
    num_rows, num_q_heads, head_dim = query.shape
    num_kv_heads = kv_cache.shape[2]
    group = num_q_heads // num_kv_heads
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    pos = [int(p) for p in positions]
    out = torch.zeros((num_rows, num_q_heads, head_dim), dtype=torch.float32)
    if not pos:
        return out
    k, v = gather_paged_kv(kv_cache, block_table, max(pos) + 1)
    k = k.repeat_interleave(group, dim=0)
    v = v.repeat_interleave(group, dim=0)
    q = query.float()
    for r, p in enumerate(pos):
        scores = torch.matmul(q[r].unsqueeze(1), k[:, :p + 1, :].transpose(-2, -1)) * scale
        out[r] = torch.matmul(torch.softmax(scores, dim=-1), v[:, :p + 1, :]).squeeze(1)
    return out


# ------------------------------------------------------------------------------------------
# Projection and orchestrator
# ------------------------------------------------------------------------------------------

def masked_qkv_projection(hidden_states, qkv_weight, compute_mask, qkv_bias=None):
    """triton_kernels.py:511-520: fp32 linear, reuse rows zeroed, cast to the input dtype."""
    projected = torch.nn.functional.linear(
        hidden_states.float(), qkv_weight.float(),
        qkv_bias.float() if qkv_bias is not None else None)
    return (projected * compute_mask.unsqueeze(1).float()).to(hidden_states.dtype)


def qkv_project_paged(hidden_states, qkv_weight, positions, kv_cache, block_table, num_heads,
                      num_kv_heads, head_dim, qkv_bias=None, rope_base=None):
    """Compacted, GQA form of the masked projection (triton_kernels.py:511-520: fp32 linear,
    one rounding to the input dtype) restricted to the rows at ``positions``, with the new
    K/V written into the paged cache at those positions.

    Features are laid out Q [Hq*D] | K [Hkv*D] | V [Hkv*D]. With ``rope_base``, Q and K of
    the row at position p are rotated in fp32 by p with the path's interleaved RoPE
    (rope_correction.py:163-178, angle ``float(p) * inv_freq``) before the rounding. K/V rows
    whose paged slot is out of range are not written; rows whose position lies outside the
    hidden states give zero Q and write nothing. Returns Q [R, Hq, D] in the input dtype.
    """
    seq_len = hidden_states.shape[0]
    pos = torch.as_tensor(positions).long()
    n = pos.shape[0]
    valid = (pos >= 0) & (pos < seq_len)
    x = torch.zeros((n, hidden_states.shape[1]), dtype=torch.float32)
    x[valid] = hidden_states[pos[valid]].float()
    proj = torch.nn.functional.linear(x, qkv_weight.float(),
                                      qkv_bias.float() if qkv_bias is not None else None)
    qf, kf = num_heads * head_dim, num_kv_heads * head_dim
    q = proj[:, :qf].reshape(n, num_heads, head_dim)
    k = proj[:, qf:qf + kf].reshape(n, num_kv_heads, head_dim)
    v = proj[:, qf + kf:qf + 2 * kf].reshape(n, num_kv_heads, head_dim)
    if rope_base is not None:
        theta = pos.to(torch.float32)[:, None] * inv_freq(rope_base, head_dim)[None, :]
        c, s = torch.cos(theta)[:, None, :], torch.sin(theta)[:, None, :]
        q = rotate_interleaved(q, c, s)
        k = rotate_interleaved(k, c, s)
    q[~valid] = 0.0
    num_blocks_total, _, _, block_size, _ = kv_cache.shape
    for r in range(n):
        if not bool(valid[r]):
            continue
        slot = _paged_slot(block_table, int(pos[r]), block_size, num_blocks_total)
        if slot is None:
            continue
        kv_cache[slot[0], 0, :, slot[1], :] = k[r].to(kv_cache.dtype)
        kv_cache[slot[0], 1, :, slot[1], :] = v[r].to(kv_cache.dtype)
    return q.to(hidden_states.dtype)


def partial_prefill(hidden_states, donor_kv, qkv_weight, output_projection, donor_positions,
                    target_positions, compute_mask, num_heads, head_dim, qkv_bias=None,
                    output_bias=None, scale=None):
    """triton_kernels.py:809-923 without timing: returns (output, target_kv, computed, reused,
    ratio)."""
    seq_len = hidden_states.shape[0]
    num_layers = donor_kv.shape[0]
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    target_kv = torch.zeros((num_layers, 2, num_heads, seq_len, head_dim),
                            dtype=hidden_states.dtype)
    scatter_donor_kv(target_kv, donor_kv, donor_positions, target_positions)
    qkv = masked_qkv_projection(hidden_states, qkv_weight, compute_mask, qkv_bias)
    qkv = qkv.float().view(seq_len, 3, num_heads, head_dim)
    q_new = qkv[:, 0].permute(1, 0, 2)
    k_new = qkv[:, 1].permute(1, 0, 2)
    v_new = qkv[:, 2].permute(1, 0, 2)
    compute_idx = torch.where(compute_mask)[0]
    reuse_idx = torch.where(~compute_mask)[0]
    merged_k = target_kv[0, 0].float().clone()
    merged_v = target_kv[0, 1].float().clone()
    if compute_idx.numel():
        merged_k[:, compute_idx, :] = k_new[:, compute_idx, :]
        merged_v[:, compute_idx, :] = v_new[:, compute_idx, :]
    attn = partial_prefill_attention(q_new, merged_k, merged_v, compute_mask, scale)
    flat = attn.permute(1, 0, 2).reshape(seq_len, num_heads * head_dim)
    out = torch.nn.functional.linear(
        flat, output_projection.float(),
        output_bias.float() if output_bias is not None else None).to(hidden_states.dtype)
    if reuse_idx.numel():
        out[reuse_idx] = 0.0
    for layer in range(num_layers):
        if compute_idx.numel():
            target_kv[layer, 0, :, compute_idx, :] = k_new[:, compute_idx, :].to(target_kv.dtype)
            target_kv[layer, 1, :, compute_idx, :] = v_new[:, compute_idx, :].to(target_kv.dtype)
    computed = int(compute_mask.sum())
    return out, target_kv, computed, seq_len - computed, computed / seq_len if seq_len else 1.0
