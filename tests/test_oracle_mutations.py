"""Planted mistakes in copies of the oracle must each be caught by a pinning check.

Every mutant below is a plausible implementation error (wrong rotation convention, wrong sign,
wrong frequency exponent, off-by-one causal bound, missing scale, wrong GQA head mapping,
ignored block table, swapped pair roles, snapshot instead of sequential V copies, fp16 storage
of K). A mutant passes this test only if at least one check in tests/pinning.py rejects it,
which shows the checks pin the oracle rather than restate it. CPU only.
"""

from __future__ import annotations

import math
import types

import pytest
import torch

from oracle import ref_cpu as ref
from tests import pinning

API = [
    "apply_rope_delta_inplace", "composite_scatter_paged", "masked_qkv_projection", "nope_permute_paged_kv",
    "partial_attention_paged", "partial_prefill", "partial_prefill_attention",
    "permute_paged_kv_with_rope", "qkv_project_paged", "rope_correct_k",
    "rope_correct_scatter_paged",
    "scatter_donor_kv", "scatter_donor_kv_paged",
]


def _ns(**overrides):
    ns = types.SimpleNamespace(**{n: getattr(ref, n) for n in API})
    for k, v in overrides.items():
        setattr(ns, k, v)
    return ns


def _failures(impl) -> list[str]:
    caught = []
    for check in pinning.ALL_CHECKS:
        try:
            check(impl)
        except Exception as exc:  # noqa: BLE001 - any failure counts as detection
            caught.append(f"{check.__name__}: {type(exc).__name__}")
    return caught


# ---- mutants of shared RoPE helpers (patched in the oracle module) ----

def _rotate_neox(k, cos, sin):
    k = k.float()
    half = k.shape[-1] // 2
    x1, x2 = k[..., :half], k[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1)


def _interleaved(k, cos, sin):
    k = k.float()
    out = torch.zeros_like(k)
    out[..., 0::2] = k[..., 0::2] * cos - k[..., 1::2] * sin
    out[..., 1::2] = k[..., 0::2] * sin + k[..., 1::2] * cos
    return out


def _inv_freq_wrong_exponent(rope_base, head_dim):
    return 1.0 / (rope_base ** (torch.arange(0, head_dim // 2, dtype=torch.float32) / head_dim))


def _rotate_store_fp16(k, cos, sin):
    return _interleaved(k, cos, sin).half().float()


HELPER_MUTANTS = {
    "neox_rotate_half": ("rotate_interleaved", _rotate_neox),
    "negated_sin": ("rotate_interleaved", lambda k, c, s: _interleaved(k, c, -s)),
    "inv_freq_i_over_d": ("inv_freq", _inv_freq_wrong_exponent),
    "k_stored_as_fp16": ("rotate_interleaved", _rotate_store_fp16),
}


@pytest.mark.parametrize("name", sorted(HELPER_MUTANTS))
def test_helper_mutant_is_caught(monkeypatch, name):
    attr, fn = HELPER_MUTANTS[name]
    monkeypatch.setattr(ref, attr, fn)
    caught = _failures(_ns())
    assert caught, f"mutant {name} passed every pinning check"


# ---- mutants of whole functions ----

def _rope_k_delta_reversed(k, d, t, head_dim=128, rope_base=10000.0):
    return ref.rope_correct_k(k, d, 2 * d - t, head_dim=head_dim, rope_base=rope_base)


def _attn_off_by_one(query, key, value, compute_mask, scale=None):
    h, s, d = query.shape
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = torch.zeros((h, s, d))
    for pos in torch.where(compute_mask.bool())[0].tolist():
        n = max(pos, 1)  # attends to keys 0..pos-1 (key 0 alone for pos 0)
        w = torch.softmax(query[:, pos:pos + 1].float() @ key[:, :n].float().transpose(-2, -1)
                          * scale, dim=-1)
        out[:, pos:pos + 1] = w @ value[:, :n].float()
    return out


def _attn_no_scale(query, key, value, compute_mask, scale=None):
    return ref.partial_prefill_attention(query, key, value, compute_mask, 1.0)


def _gqa_modulo_heads(query, kv_cache, block_table, positions, scale=None):
    hq, hkv = query.shape[1], kv_cache.shape[2]
    # head h reads kv head h % hkv instead of h // (hq // hkv)
    perm = torch.tensor([(h % hkv) * (hq // hkv) + h // hkv for h in range(hq)])
    inv = torch.argsort(perm)
    out = ref.partial_attention_paged(query[:, inv], kv_cache, block_table, positions, scale)
    return out[:, perm]


def _paged_scatter_ignores_table(kv_cache, donor_kv, block_table, dpos, tpos):
    ident = torch.arange(max(block_table.shape[0], kv_cache.shape[0]), dtype=torch.int32)
    return ref.scatter_donor_kv_paged(kv_cache, donor_kv, ident[: block_table.shape[0]], dpos,
                                      tpos)


def _scatter_swapped(target, donor, dpos, tpos):
    return ref.scatter_donor_kv(target, donor, tpos, dpos)


def _nope_snapshot_v(kv_cache, block_table, permutation, rope_base=10000.0):
    bs = kv_cache.shape[3]
    snaps = []
    for s, t in permutation:
        sb = int(block_table[s // bs])
        snaps.append((t, kv_cache[sb, 1, :, s % bs].clone()))
    saved = kv_cache[:, 1].clone()
    ref.nope_permute_paged_kv(kv_cache, block_table, permutation, rope_base)
    kv_cache[:, 1] = saved
    for t, v in snaps:
        kv_cache[int(block_table[t // bs]), 1, :, t % bs] = v



def _composite_donor_ignored(kv_cache, donor_kvs, block_table, didx, dpos, tpos, rope=True,
                             rope_base=10000.0):
    # every pair read from the first donor
    valid = (torch.as_tensor(didx) >= 0) & (torch.as_tensor(didx) < len(donor_kvs))
    return ref.composite_scatter_paged(kv_cache, donor_kvs[:1], block_table,
                                       torch.where(valid, 0, -1), dpos, tpos, rope, rope_base)


def _composite_last_donor_dropped(kv_cache, donor_kvs, block_table, didx, dpos, tpos,
                                  rope=True, rope_base=10000.0):
    return ref.composite_scatter_paged(kv_cache, donor_kvs[:-1], block_table, didx, dpos, tpos,
                                       rope, rope_base)


def _composite_rope_dropped(kv_cache, donor_kvs, block_table, didx, dpos, tpos, rope=True,
                            rope_base=10000.0):
    return ref.composite_scatter_paged(kv_cache, donor_kvs, block_table, didx, dpos, tpos, False,
                                       rope_base)



def _proj_kv_swapped(hs, w, pos, kv_cache, bt, h, hkv, d, qkv_bias=None, rope_base=None):
    qf, kf = h * d, hkv * d
    w2 = torch.cat([w[:qf], w[qf + kf:], w[qf:qf + kf]])
    b2 = None if qkv_bias is None else torch.cat(
        [qkv_bias[:qf], qkv_bias[qf + kf:], qkv_bias[qf:qf + kf]])
    return ref.qkv_project_paged(hs, w2, pos, kv_cache, bt, h, hkv, d, b2, rope_base)


def _proj_kv_interleaved_per_head(hs, w, pos, kv_cache, bt, h, hkv, d, qkv_bias=None,
                                  rope_base=None):
    # reads the K/V rows as [K0 V0 K1 V1 ...] instead of [K0 K1 ... V0 V1 ...]
    qf, kf = h * d, hkv * d
    kv_rows = w[qf:qf + 2 * kf].reshape(hkv, 2, d, -1)
    w2 = torch.cat([w[:qf], kv_rows[:, 0].reshape(kf, -1), kv_rows[:, 1].reshape(kf, -1)])
    b2 = qkv_bias
    if qkv_bias is not None:
        kb = qkv_bias[qf:qf + 2 * kf].reshape(hkv, 2, d)
        b2 = torch.cat([qkv_bias[:qf], kb[:, 0].reshape(-1), kb[:, 1].reshape(-1)])
    return ref.qkv_project_paged(hs, w2, pos, kv_cache, bt, h, hkv, d, b2, rope_base)


def _proj_rope_on_v(hs, w, pos, kv_cache, bt, h, hkv, d, qkv_bias=None, rope_base=None):
    q = ref.qkv_project_paged(hs, w, pos, kv_cache, bt, h, hkv, d, qkv_bias, rope_base)
    if rope_base is not None:
        bs = kv_cache.shape[3]
        f = ref.inv_freq(rope_base, d)
        for p in torch.as_tensor(pos).tolist():
            if 0 <= p // bs < bt.shape[0]:
                pb, off = int(bt[p // bs]), p % bs
                th = float(p) * f
                kv_cache[pb, 1, :, off] = ref.rotate_interleaved(
                    kv_cache[pb, 1, :, off], torch.cos(th), torch.sin(th)).to(kv_cache.dtype)
    return q


def _proj_rope_q_skipped(hs, w, pos, kv_cache, bt, h, hkv, d, qkv_bias=None, rope_base=None):
    ref.qkv_project_paged(hs, w, pos, kv_cache, bt, h, hkv, d, qkv_bias, rope_base)
    return ref.qkv_project_paged(hs, w, pos, kv_cache.clone(), bt, h, hkv, d, qkv_bias, None)


def _prefill_mutant(kind):
    """The orchestrator (triton_kernels.py:809-923) with one planted mistake of ``kind``."""

    def run(hidden_states, donor_kv, qkv_weight, output_projection, donor_positions,
            target_positions, compute_mask, num_heads, head_dim, qkv_bias=None,
            output_bias=None, scale=None):
        seq, layers = hidden_states.shape[0], donor_kv.shape[0]
        h, d = num_heads, head_dim
        scale = 1.0 / math.sqrt(d) if scale is None else scale
        target = torch.zeros((layers, 2, h, seq, d), dtype=hidden_states.dtype)
        ref.scatter_donor_kv(target, donor_kv, donor_positions, target_positions)
        qkv = ref.masked_qkv_projection(hidden_states, qkv_weight, compute_mask, qkv_bias).float()
        if kind == "heads_major_split":
            qkv = qkv.view(seq, h, 3, d)
            q_new, k_new, v_new = (qkv[:, :, i].permute(1, 0, 2) for i in range(3))
        else:
            qkv = qkv.view(seq, 3, h, d)
            q_new, k_new, v_new = (qkv[:, i].permute(1, 0, 2) for i in range(3))
        comp = torch.where(compute_mask)[0]
        src_layer = layers - 1 if kind == "last_layer_attention" else 0
        mk = target[src_layer, 0].float().clone()
        mv = target[src_layer, 1].float().clone()
        if kind != "new_kv_not_merged":
            mk[:, comp] = k_new[:, comp]
            mv[:, comp] = v_new[:, comp]
        attn = ref.partial_prefill_attention(q_new, mk, mv, compute_mask, scale)
        flat = attn.permute(1, 0, 2).reshape(seq, h * d)
        wo = output_projection.float()
        if kind == "output_projection_transposed":
            wo = wo.t()
        out = torch.nn.functional.linear(
            flat, wo, output_bias.float() if output_bias is not None else None)
        out = out.to(hidden_states.dtype)
        out[torch.where(~compute_mask)[0]] = 0.0
        kw, vw = (v_new, k_new) if kind == "kv_swapped_in_writeback" else (k_new, v_new)
        for layer in range(layers):
            target[layer, 0, :, comp] = kw[:, comp].to(target.dtype)
            target[layer, 1, :, comp] = vw[:, comp].to(target.dtype)
        computed = int(compute_mask.sum())
        return out, target, computed, seq - computed, computed / seq if seq else 1.0

    return run


FUNCTION_MUTANTS = {
    "rope_delta_reversed": {"rope_correct_k": _rope_k_delta_reversed},
    "attention_causal_off_by_one": {"partial_prefill_attention": _attn_off_by_one},
    "attention_scale_dropped": {"partial_prefill_attention": _attn_no_scale},
    "gqa_head_mapping_modulo": {"partial_attention_paged": _gqa_modulo_heads},
    "paged_scatter_ignores_block_table": {"scatter_donor_kv_paged": _paged_scatter_ignores_table},
    "scatter_pair_roles_swapped": {"scatter_donor_kv": _scatter_swapped},
    "nope_v_snapshot_instead_of_sequential": {"nope_permute_paged_kv": _nope_snapshot_v},
    "composite_donor_index_ignored": {"composite_scatter_paged": _composite_donor_ignored},
    "composite_last_donor_dropped": {"composite_scatter_paged": _composite_last_donor_dropped},
    "composite_rope_dropped": {"composite_scatter_paged": _composite_rope_dropped},
    "projection_k_v_swapped": {"qkv_project_paged": _proj_kv_swapped},
    "projection_kv_interleaved_per_head": {"qkv_project_paged": _proj_kv_interleaved_per_head},
    "projection_rope_on_v": {"qkv_project_paged": _proj_rope_on_v},
    "projection_rope_q_skipped": {"qkv_project_paged": _proj_rope_q_skipped},
    **{f"prefill_{k}": {"partial_prefill": _prefill_mutant(k)}
       for k in ("heads_major_split", "new_kv_not_merged", "last_layer_attention",
                 "output_projection_transposed", "kv_swapped_in_writeback")},
}


def test_prefill_mutant_harness_is_faithful():
    """The mutant harness with no mistake planted passes every check (so each mutant's
    failure comes from its planted mistake)."""
    assert _failures(_ns(partial_prefill=_prefill_mutant("none"))) == []


@pytest.mark.parametrize("name", sorted(FUNCTION_MUTANTS))
def test_function_mutant_is_caught(name):
    caught = _failures(_ns(**FUNCTION_MUTANTS[name]))
    assert caught, f"mutant {name} passed every pinning check"


def test_unmutated_oracle_passes_everything():
    assert _failures(_ns()) == []
