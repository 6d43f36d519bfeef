"""SemBlend partial-prefill kernels on MI355X — drop-in for ``semblend_core.triton_kernels``
(semblend_core/triton_kernels.py).

The module keeps the reference's names, signatures, defaults and return conventions:

* ``scatter_donor_kv`` / ``scatter_donor_kv_paged`` — donor KV copied into the target cache,
  in place, bit-exact (HIP row mover, 16-byte vector loads);
* ``masked_qkv_projection`` — projection for compute rows only, reuse rows zero (bf16/fp16:
  a compacted MFMA GEMM over the computed rows only; fp32: torch's GEMM, as the reference);
* ``partial_prefill_attention`` — causal attention for compute rows only, zero elsewhere
  (bf16/fp16 MFMA kernel with an fp32 online softmax; fp32 inputs take an fp32 kernel);
* ``partial_prefill`` / ``PartialPrefillResult`` — the single-layer orchestrator.

Extensions with no reference counterpart: ``scatter_donor_kv_paged_layers`` (many layers in
one launch), ``partial_prefill_attention_paged`` (GQA over a paged cache for a compact set of
query rows) and ``qkv_projection_paged`` (compacted GQA projection that writes the new K/V
into the paged cache, optionally with RoPE at the new positions), and
``partial_prefill_layer_paged``, one attention layer of partial prefill over a paged cache
built from those pieces. CPU tensors are rejected: the kernels exist only for HIP devices.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import _lib

# Import-compatibility flag (the reference exports it, semblend_core/triton_kernels.py:42-50).
# There is no Triton here; HAS_HIP reports whether the HIP kernel library loaded.
HAS_TRITON = False
HAS_HIP = _lib.available()

__all__ = [
    "HAS_TRITON",
    "HAS_HIP",
    "PartialPrefillResult",
    "masked_qkv_projection",
    "partial_prefill",
    "partial_prefill_attention",
    "partial_prefill_attention_paged",
    "plan_partial_attention_paged",
    "PagedAttentionPlan",
    "partial_prefill_layer_paged",
    "PagedLayerResult",
    "qkv_projection_paged",
    "scatter_donor_kv",
    "scatter_donor_kv_paged",
    "scatter_donor_kv_paged_layers",
]


# ------------------------------------------------------------------------------------------
# Donor-KV scatter
# ------------------------------------------------------------------------------------------

def _check_pair_lengths(donor_positions, target_positions) -> int:
    """Number of (donor, target) pairs; the two position lists must have the same length
    (the kernels read one target per donor position)."""
    n = len(donor_positions)
    if len(target_positions) != n:
        raise ValueError(f"donor_positions ({n}) and target_positions "
                         f"({len(target_positions)}) differ in length")
    return n


def _contig_last(t: torch.Tensor) -> tuple[torch.Tensor, bool]:
    """(tensor with unit stride in the last dim, whether it is a temporary copy)."""
    if t.stride(-1) == 1:
        return t, False
    return t.contiguous(), True


def scatter_donor_kv(
    target: torch.Tensor,
    donor: torch.Tensor,
    donor_positions: torch.Tensor,
    target_positions: torch.Tensor,
) -> torch.Tensor:
    """``target[:, :, :, t, :] = donor[:, :, :, d, :]`` for every (d, t) pair, all layers.

    target: [num_layers, 2, num_heads, target_seq_len, head_dim];
    donor:  [num_layers, 2, num_heads, donor_seq_len, head_dim].
    Pairs with d >= donor_seq_len or t >= target_seq_len (or negative) are skipped.
    Returns target (modified in place). Reference: semblend_core/triton_kernels.py:132-191.
    """
    num_pairs = _check_pair_lengths(donor_positions, target_positions)
    if num_pairs == 0:
        return target
    dev = _lib.require_device(target, donor)
    if target.dtype != donor.dtype:
        raise TypeError("target and donor must share a dtype")
    num_layers, _, num_heads, target_seq_len, head_dim = target.shape
    donor_seq_len = donor.shape[3]
    dpos = _lib.as_index(donor_positions, dev)
    tpos = _lib.as_index(target_positions, dev)
    tw, t_tmp = _contig_last(target)
    dw, _ = _contig_last(donor)
    with _lib.on_device(dev):
        _lib.call(
            "sb_scatter_donor_kv",
            tw.data_ptr(), dw.data_ptr(), dpos.data_ptr(), tpos.data_ptr(), num_pairs,
            num_layers, num_heads, head_dim, target_seq_len, donor_seq_len, _lib.strides(tw),
            _lib.strides(dw), _lib.dtype_code(tw), _lib.stream_handle(dev),
        )
    if t_tmp:
        target.copy_(tw)
    return target


def scatter_donor_kv_paged(
    kv_cache: torch.Tensor,
    donor_kv: torch.Tensor,
    block_table: torch.Tensor,
    donor_positions: torch.Tensor,
    target_positions: torch.Tensor,
) -> torch.Tensor:
    """``kv_cache[bt[t // bs], :, :, t % bs, :] = donor_kv[:, :, d, :]`` for every pair.

    kv_cache: [num_blocks, 2, num_heads, block_size, head_dim] (any strides);
    donor_kv: [2, num_heads, donor_seq_len, head_dim]; block_table: [num_blocks_per_seq].
    Pairs whose donor position, logical block or physical block is out of range are skipped
    (the reference GPU kernel's rule, semblend_core/triton_kernels.py:246-260).
    Returns kv_cache (modified in place). Reference: semblend_core/triton_kernels.py:279-356.
    """
    num_pairs = _check_pair_lengths(donor_positions, target_positions)
    if num_pairs == 0:
        return kv_cache
    dev = _lib.require_device(kv_cache, donor_kv)
    if kv_cache.dtype != donor_kv.dtype:
        raise TypeError("kv_cache and donor_kv must share a dtype")
    nb_total, _, num_heads, block_size, head_dim = kv_cache.shape
    bt = _lib.as_index(block_table, dev)
    dpos = _lib.as_index(donor_positions, dev)
    tpos = _lib.as_index(target_positions, dev)
    kw, k_tmp = _contig_last(kv_cache)
    dw, _ = _contig_last(donor_kv)
    with _lib.on_device(dev):
        _lib.call(
            "sb_scatter_donor_kv_paged",
            kw.data_ptr(), dw.data_ptr(), bt.data_ptr(), dpos.data_ptr(), tpos.data_ptr(),
            num_pairs, num_heads, block_size, head_dim, dw.shape[2], nb_total, bt.shape[0],
            _lib.strides(kw), _lib.strides(dw), _lib.dtype_code(kw), _lib.stream_handle(dev),
        )
    if k_tmp:
        kv_cache.copy_(kw)
    return kv_cache


def scatter_donor_kv_paged_layers(
    kv_caches: list[torch.Tensor],
    donor_kvs: list[torch.Tensor],
    block_table: torch.Tensor,
    donor_positions: torch.Tensor,
    target_positions: torch.Tensor,
    repeated_donor_rows: bool | None = None,
) -> list[torch.Tensor]:
    """``scatter_donor_kv_paged`` for every layer in a single launch.

    kv_caches / donor_kvs: one tensor per layer (same shape, strides and dtype across
    layers, 16-byte aligned bases). repeated_donor_rows: whether a donor position may be the
    source of several pairs (the donor is then read through the caches); None decides from
    host positions and takes device positions as distinct. It changes speed, not results.
    Extension with no reference counterpart; it replaces the per-layer Python loop of callers
    such as synapse_kv_connector/model_runner_hook.py:215-276.
    """
    if len(kv_caches) != len(donor_kvs):
        raise ValueError("kv_caches and donor_kvs must have the same length")
    num_pairs = _check_pair_lengths(donor_positions, target_positions)
    if num_pairs == 0 or not kv_caches:
        return kv_caches
    dev = _lib.require_device(*kv_caches, *donor_kvs)
    ref, dref = kv_caches[0], donor_kvs[0]
    for group, name in ((kv_caches, "kv_caches"), (donor_kvs, "donor_kvs")):
        for t in group:
            if t.shape != group[0].shape or t.stride() != group[0].stride() or \
                    t.dtype != group[0].dtype:
                raise ValueError(f"all {name} must share shape, strides and dtype")
            if t.data_ptr() % 16 or t.stride(-1) != 1:
                raise ValueError(f"{name} need 16-byte aligned bases and unit last stride")
    if ref.dtype != dref.dtype:
        raise TypeError("kv_caches and donor_kvs must share a dtype")
    nb_total, _, num_heads, block_size, head_dim = ref.shape
    if repeated_donor_rows is None:
        repeated_donor_rows = _lib.rows_repeat(donor_positions)
    kv_tab = _lib.address_table(kv_caches, dev)
    d_tab = _lib.address_table(donor_kvs, dev)
    bt = _lib.as_index(block_table, dev)
    dpos = _lib.as_index(donor_positions, dev)
    tpos = _lib.as_index(target_positions, dev)
    with _lib.on_device(dev):
        _lib.call(
            "sb_scatter_donor_kv_paged_layers",
            kv_tab.data_ptr(), d_tab.data_ptr(), len(kv_caches), bt.data_ptr(),
            dpos.data_ptr(), tpos.data_ptr(), num_pairs, num_heads, block_size, head_dim,
            dref.shape[2], nb_total, bt.shape[0], _lib.strides(ref), _lib.strides(dref),
            _lib.dtype_code(ref), _lib.scatter_flags(repeated_donor_rows),
            _lib.stream_handle(dev),
        )
    return kv_caches


# ------------------------------------------------------------------------------------------
# Masked QKV projection
# ------------------------------------------------------------------------------------------

def _mfma_rows_ok(*ts: torch.Tensor) -> bool:
    """Row-major 2-D operands the MFMA projection can stream (16-byte aligned rows)."""
    return all(t.dim() == 2 and t.stride(1) == 1 and t.data_ptr() % 16 == 0
               and (t.stride(0) * t.element_size()) % 16 == 0 for t in ts)


def masked_qkv_projection(
    hidden_states: torch.Tensor,
    qkv_weight: torch.Tensor,
    compute_mask: torch.Tensor,
    qkv_bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """QKV projection whose reuse rows (compute_mask == False) are zero.

    hidden_states [seq_len, hidden]; qkv_weight [3 * H * D, hidden]; output
    [seq_len, 3 * H * D] in the input dtype, accumulated in fp32 and rounded once (the
    reference projects in fp32 and casts back, semblend_core/triton_kernels.py:511-520).
    bf16 / fp16 with a hidden size that is a multiple of 64 run ``sb_masked_qkv_projection``:
    the mask is compacted on the device and only the computed rows are multiplied (MFMA);
    other cases run torch's GEMM in fp32 on the device, as the reference's fallback does.
    Reference: :451-522.
    """
    dev = _lib.require_device(hidden_states, qkv_weight)
    seq_len, hidden = hidden_states.shape
    out_features = qkv_weight.shape[0]
    dt = hidden_states.dtype
    mask = compute_mask.to(device=dev)
    if (dt in (torch.bfloat16, torch.float16) and qkv_weight.dtype == dt
            and (qkv_bias is None or qkv_bias.dtype == dt) and hidden % 64 == 0
            and out_features % 8 == 0 and seq_len > 0
            and _mfma_rows_ok(hidden_states, qkv_weight)):
        out = torch.empty((seq_len, out_features), dtype=dt, device=dev)
        mask_u8 = (mask if mask.dtype == torch.bool else mask != 0).contiguous().view(torch.uint8)
        bias = None if qkv_bias is None else qkv_bias.contiguous()
        ws_bytes = _lib.size_query("sb_masked_qkv_projection_workspace_size", seq_len)
        ws = torch.empty(ws_bytes // 4, dtype=torch.int32, device=dev)
        with _lib.on_device(dev):
            _lib.call(
                "sb_masked_qkv_projection",
                out.data_ptr(), hidden_states.data_ptr(), qkv_weight.data_ptr(), _lib.ptr(bias),
                mask_u8.data_ptr(), ws.data_ptr(), ws_bytes, seq_len, hidden, out_features,
                hidden_states.stride(0), qkv_weight.stride(0), out.stride(0),
                _lib.dtype_code(hidden_states), _lib.stream_handle(dev),
            )
        return out
    projected = torch.nn.functional.linear(
        hidden_states.float(),
        qkv_weight.float(),
        qkv_bias.float() if qkv_bias is not None else None,
    )
    return (projected * mask.unsqueeze(1).float()).to(dt)




# Row counts in which qkv_projection_paged(backend="auto") takes the library GEMM (measured at
# the Qwen2.5-7B shape: the fused kernel is faster or level below and above this range).
_LIBRARY_PROJECTION_ROWS = (513, 1024)


def qkv_projection_paged(
    hidden_states: torch.Tensor,
    qkv_weight: torch.Tensor,
    positions: torch.Tensor,
    kv_cache: torch.Tensor,
    block_table: torch.Tensor,
    num_heads: int,
    num_kv_heads: int,
    head_dim: int,
    qkv_bias: torch.Tensor | None = None,
    rope_base: float | None = None,
    out: torch.Tensor | None = None,
    backend: str = "auto",
) -> torch.Tensor:
    """Project only the rows at ``positions`` and write their new K/V into the paged cache.

    hidden_states [S, hidden]; qkv_weight [(Hq + 2 * Hkv) * D, hidden] with features laid out
    Q | K | V (+ qkv_bias of the same length); kv_cache [NB, 2, Hkv, bs, D] with its block
    table. Returns Q [R, Hq, D] for the computed rows (``out`` may supply it). With
    ``rope_base``, Q and K are rotated by their position with the interleaved RoPE of this
    path before the single rounding. K/V slots out of the table are skipped; a position
    outside the hidden states gives a zero Q row. bf16 / fp16, head_dim a multiple of 8,
    hidden a multiple of 64 for the fused form and of 8 for the library form.
    ``backend``: "fused" runs one MFMA kernel that gathers the rows, multiplies and writes
    Q and K/V from its epilogue; "library" gathers the rows, multiplies them with the
    library GEMM (hipBLASLt through torch, fp32 output) and runs the same epilogue as a
    kernel of its own (bias, RoPE, one rounding, Q and the paged K/V write); "auto" takes the
    library form from 513 to 1024 rows and the fused form otherwise (which splits the hidden
    dimension when its row tiles are too few for the CUs). Qwen2.5-7B shape, graph replays on
    one MI355X, fused / library: 28.5 / 28 us at 64 rows, 36.5 / 46 at 256, 42.5 / 43.5 at
    512, 52 / 48 at 768, 57 / 56.5 at 1024, 83 / 86.5 at 2048, 89 / 98 at 2458, 158 / 165 at
    4096. The fused form needs no fp32 intermediate of rows x features. Both accumulate in
    fp32 and round once.
    Fuses the masked projection (semblend_core/triton_kernels.py:451-522) with the K/V write
    of partial_prefill (:904-909), compacted and paged; no reference counterpart.
    """
    from .rope_correction import inv_freq_table

    if backend not in ("auto", "fused", "library"):
        raise ValueError("backend must be 'auto', 'fused' or 'library'")
    dev = _lib.require_device(hidden_states, qkv_weight, kv_cache)
    dt = hidden_states.dtype
    if dt not in (torch.bfloat16, torch.float16):
        raise TypeError("qkv_projection_paged runs bf16 / fp16 (the MFMA path)")
    if qkv_weight.dtype != dt or kv_cache.dtype != dt or (
            qkv_bias is not None and qkv_bias.dtype != dt):
        raise TypeError("hidden_states, qkv_weight, qkv_bias and kv_cache must share a dtype")
    seq_len, hidden = hidden_states.shape
    features = (num_heads + 2 * num_kv_heads) * head_dim
    if qkv_weight.shape != (features, hidden):
        raise ValueError(f"qkv_weight must be [{features}, {hidden}]")
    if qkv_bias is not None and qkv_bias.shape != (features,):
        raise ValueError(f"qkv_bias must be [{features}]")
    nb, two, hkv, bs, d = kv_cache.shape
    if two != 2 or hkv != num_kv_heads or d != head_dim:
        raise ValueError("kv_cache must be [num_blocks, 2, num_kv_heads, block_size, head_dim]")
    if not _mfma_rows_ok(hidden_states, qkv_weight):
        raise ValueError("hidden_states and qkv_weight need unit-stride, 16-byte aligned rows")
    pos = _lib.as_index(positions, dev)
    bt = _lib.as_index(block_table, dev)
    n = pos.shape[0]
    if out is None:
        out = torch.empty((n, num_heads, head_dim), dtype=dt, device=dev)
    elif out.shape != (n, num_heads, head_dim) or out.dtype != dt or not out.is_contiguous():
        raise ValueError("out must be a contiguous [R, Hq, D] tensor of the input dtype")
    if n == 0:
        return out
    bias = None if qkv_bias is None else qkv_bias.contiguous()
    inv = inv_freq_table(rope_base, head_dim, dev) if rope_base is not None else None
    if backend == "auto":
        lo, hi = _LIBRARY_PROJECTION_ROWS
        backend = "library" if lo <= n <= hi else "fused"
    if backend == "library":
        # rows outside the hidden states are gathered as zeros; the epilogue zeroes their Q
        # and writes no K/V for them
        xg = torch.empty((n, hidden), dtype=dt, device=dev)
        ws = torch.empty(max(n * head_dim, 4) if inv is not None else 4, dtype=torch.float32,
                         device=dev)
        dt_code = _lib.dtype_code(hidden_states)
        with _lib.on_device(dev):
            _lib.call("sb_qkv_gather_rows", xg.data_ptr(), hidden_states.data_ptr(),
                      pos.data_ptr(), n, seq_len, hidden, hidden_states.stride(0),
                      _lib.ptr(inv), head_dim, ws.data_ptr(), dt_code, _lib.stream_handle(dev))
            proj = torch.mm(xg, qkv_weight.t(), out_dtype=torch.float32)
            _lib.call(
                "sb_qkv_epilogue_paged",
                out.data_ptr(), proj.data_ptr(), _lib.ptr(bias), pos.data_ptr(), n, seq_len,
                num_heads, num_kv_heads, head_dim, ws.data_ptr() if inv is not None else None,
                kv_cache.data_ptr(), bt.data_ptr(), bs, nb, bt.shape[0], proj.stride(0),
                num_heads * head_dim, _lib.strides(kv_cache), dt_code, _lib.stream_handle(dev),
            )
        return out
    ws_bytes = _lib.size_query("sb_qkv_projection_paged_workspace_size", n, num_heads,
                               num_kv_heads, head_dim, hidden, int(inv is not None))
    ws = torch.empty(max(ws_bytes, 16) // 4, dtype=torch.float32, device=dev)
    with _lib.on_device(dev):
        _lib.call(
            "sb_qkv_projection_paged",
            out.data_ptr(), hidden_states.data_ptr(), qkv_weight.data_ptr(), _lib.ptr(bias),
            pos.data_ptr(), n, seq_len, hidden, num_heads, num_kv_heads, head_dim,
            _lib.ptr(inv), ws.data_ptr(), ws_bytes, kv_cache.data_ptr(), bt.data_ptr(), bs, nb,
            bt.shape[0],
            hidden_states.stride(0), qkv_weight.stride(0), num_heads * head_dim,
            _lib.strides(kv_cache), _lib.dtype_code(hidden_states), _lib.stream_handle(dev),
        )
    return out


# ------------------------------------------------------------------------------------------
# Partial prefill attention
# ------------------------------------------------------------------------------------------

def partial_prefill_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    compute_mask: torch.Tensor,
    scale: float | None = None,
) -> torch.Tensor:
    """Causal attention for the rows where ``compute_mask`` is True; other rows are 0.

    query, key, value: [num_heads, seq_len, head_dim]. Row i attends to keys 0..i:
    ``out[:, i] = softmax(scale * q[:, i] k[:, :i+1]^T) v[:, :i+1]`` with
    ``scale = 1/sqrt(head_dim)`` by default. fp32 accumulation for every dtype.
    The mask is compacted on the device, so the call does not synchronise with the host.
    Reference: semblend_core/triton_kernels.py:655-734.
    """
    dev = _lib.require_device(query, key, value)
    num_heads, seq_len, head_dim = query.shape
    if key.shape != query.shape or value.shape != query.shape:
        raise ValueError("query, key and value must have the same shape [H, S, D]")
    if key.dtype != query.dtype or value.dtype != query.dtype:
        raise TypeError("query, key and value must share a dtype")
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    output = torch.empty_like(query)
    if output.stride(-1) != 1:
        output = torch.empty(query.shape, dtype=query.dtype, device=dev)
    if seq_len == 0 or num_heads == 0:
        return output
    q = query if query.stride(-1) == 1 else query.contiguous()
    k = key if key.stride(-1) == 1 else key.contiguous()
    v = value if value.stride(-1) == 1 else value.contiguous()
    mask = compute_mask.to(device=dev)
    if mask.dtype != torch.bool:
        mask = mask != 0
    mask = mask.contiguous().view(torch.uint8)
    dt = _lib.dtype_code(q)
    ws_bytes = _lib.size_query("sb_partial_prefill_attention_workspace_size", num_heads,
                               seq_len, head_dim, dt)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    with _lib.on_device(dev):
        _lib.call(
            "sb_partial_prefill_attention",
            output.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), mask.data_ptr(),
            ws.data_ptr(), ws_bytes, num_heads, seq_len, head_dim, float(scale), _lib.strides(q),
            _lib.strides(k), _lib.strides(v), _lib.strides(output), _lib.dtype_code(q),
            _lib.stream_handle(dev),
        )
    return output


class PagedAttentionPlan:
    """Launch plan of :func:`partial_prefill_attention_paged` for one set of query positions
    (built by :func:`plan_partial_attention_paged`): the key split and the longest-first
    dispatch order of the work items, on the device. One request's plan serves every layer."""

    def __init__(self, num_rows, num_q_heads, num_kv_heads, head_dim, block_size,
                 num_blocks_per_seq, dtype, ks_first, ks_rest, max_chunks, order):
        self.num_rows, self.num_q_heads, self.num_kv_heads = num_rows, num_q_heads, num_kv_heads
        self.head_dim, self.block_size = head_dim, block_size
        self.num_blocks_per_seq, self.dtype = num_blocks_per_seq, dtype
        self.ks_first, self.ks_rest, self.max_chunks = ks_first, ks_rest, max_chunks
        self.order = order  # int32 device tensor (empty when the MFMA kernel does not apply)

    def matches(self, num_rows, num_q_heads, num_kv_heads, head_dim, block_size,
                num_blocks_per_seq, dtype) -> bool:
        return (self.num_rows, self.num_q_heads, self.num_kv_heads, self.head_dim,
                self.block_size, self.num_blocks_per_seq, self.dtype) == (
                    num_rows, num_q_heads, num_kv_heads, head_dim, block_size,
                    num_blocks_per_seq, dtype)


def plan_partial_attention_paged(
    compute_positions,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    block_size: int,
    num_blocks_per_seq: int,
    dtype: torch.dtype,
    device,
) -> PagedAttentionPlan:
    """Plan :func:`partial_prefill_attention_paged` for the given query positions (host data;
    a device tensor is read back once): the longest-first order in which its work items are
    dispatched, and a key split whose later chunks may be shorter than the first, chosen so
    that the last workgroups finish together. Results are correct for any positions; the plan
    makes the launch fastest for these. Extension with no reference counterpart."""
    dev = torch.device(device)
    pos = torch.as_tensor(compute_positions).reshape(-1).to("cpu", torch.int32).contiguous()
    dt = _lib.dtype_code(torch.empty(0, dtype=dtype))
    args = (ctypes.cast(pos.data_ptr(), _lib.I32P), pos.numel(),
            num_q_heads, num_kv_heads, head_dim, block_size, num_blocks_per_seq, dt)
    need = _lib.size_query("sb_partial_attention_paged_plan", *args, None, 0)
    if need < 3:
        raise RuntimeError("sb_partial_attention_paged_plan failed: "
                           + _lib.lib().sb_last_error_string().decode())
    buf = torch.empty(need, dtype=torch.int32)
    got = _lib.size_query("sb_partial_attention_paged_plan", *args,
                          ctypes.cast(buf.data_ptr(), _lib.I32P), need)
    if got != need:
        raise RuntimeError("sb_partial_attention_paged_plan failed: "
                           + _lib.lib().sb_last_error_string().decode())
    ks_first, ks_rest, max_chunks = (int(v) for v in buf[:3])
    order = buf[3:].to(dev) if need > 3 else torch.empty(0, dtype=torch.int32, device=dev)
    return PagedAttentionPlan(pos.numel(), num_q_heads, num_kv_heads, head_dim, block_size,
                              num_blocks_per_seq, dtype, ks_first, ks_rest, max_chunks, order)


def partial_prefill_attention_paged(
    query: torch.Tensor,
    kv_cache: torch.Tensor,
    block_table: torch.Tensor,
    compute_positions: torch.Tensor,
    scale: float | None = None,
    out: torch.Tensor | None = None,
    plan: PagedAttentionPlan | None = None,
) -> torch.Tensor:
    """GQA causal attention over a paged cache for a compact set of query rows.

    query: [R, num_q_heads, head_dim] — row r is the token at ``compute_positions[r]``;
    kv_cache: [num_blocks, 2, num_kv_heads, block_size, head_dim] (any strides);
    block_table: [num_blocks_per_seq]. Query head h reads KV head
    ``h // (num_q_heads // num_kv_heads)``. Returns [R, num_q_heads, head_dim]:
    ``out[r, h] = softmax(scale * q[r, h] K[0..p_r]^T) V[0..p_r]``.
    Ascending positions give the best schedule; any order is correct. Positions belong in
    ``[0, len(block_table) * block_size)``: one at or past the end attends the whole table,
    and a row with a negative position is left unwritten (no memory outside the inputs is
    touched either way).
    ``plan``: from :func:`plan_partial_attention_paged` for these positions (same row count,
    heads, head_dim, block size, table length and dtype), to launch with its split and
    longest-first order.
    Extension with no reference counterpart: the reference attention is MHA over contiguous
    K/V (semblend_core/triton_kernels.py:655-734), gathered from the cache by its callers.
    """
    dev = _lib.require_device(query, kv_cache)
    num_rows, num_q_heads, head_dim = query.shape
    nb_total, _, num_kv_heads, block_size, hd = kv_cache.shape
    if hd != head_dim:
        raise ValueError("query and kv_cache head_dim differ")
    if num_q_heads % num_kv_heads:
        raise ValueError("num_q_heads must be a multiple of num_kv_heads")
    if query.dtype != kv_cache.dtype:
        raise TypeError("query and kv_cache must share a dtype")
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    if out is None:
        out = torch.empty((num_rows, num_q_heads, head_dim), dtype=query.dtype, device=dev)
    if num_rows == 0:
        return out
    q = query if query.stride(-1) == 1 else query.contiguous()
    kv = kv_cache if kv_cache.stride(-1) == 1 else kv_cache.contiguous()
    pos = _lib.as_index(compute_positions, dev)
    if pos.shape[0] != num_rows:
        raise ValueError("compute_positions must have one entry per query row")
    bt = _lib.as_index(block_table, dev)
    dt = _lib.dtype_code(q)
    if plan is not None:
        if not plan.matches(num_rows, num_q_heads, num_kv_heads, head_dim, block_size,
                            bt.shape[0], q.dtype):
            raise ValueError("plan was made for another shape (rows, heads, head_dim, block "
                             "size, block-table length or dtype)")
        ws_bytes = _lib.size_query("sb_partial_attention_paged_planned_workspace_size",
                                   num_rows, num_q_heads, num_kv_heads, head_dim,
                                   plan.max_chunks, dt)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
        with _lib.on_device(dev):
            _lib.call(
                "sb_partial_attention_paged_planned",
                out.data_ptr(), q.data_ptr(), kv.data_ptr(), bt.data_ptr(), pos.data_ptr(),
                plan.order.data_ptr() if plan.order.numel() else None, plan.order.numel(),
                plan.ks_first, plan.ks_rest, plan.max_chunks, _lib.ptr(ws), ws_bytes, num_rows, num_q_heads,
                num_kv_heads, head_dim, block_size, nb_total, bt.shape[0], float(scale),
                _lib.strides(q), _lib.strides(out), _lib.strides(kv), dt,
                _lib.stream_handle(dev),
            )
        return out
    ws_bytes = _lib.size_query("sb_partial_attention_paged_workspace_size", num_rows,
                               num_q_heads, num_kv_heads, head_dim, block_size, bt.shape[0], dt)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    with _lib.on_device(dev):
        _lib.call(
            "sb_partial_attention_paged",
            out.data_ptr(), q.data_ptr(), kv.data_ptr(), bt.data_ptr(), pos.data_ptr(),
            _lib.ptr(ws), ws_bytes, num_rows, num_q_heads, num_kv_heads, head_dim, block_size,
            nb_total, bt.shape[0],
            float(scale), _lib.strides(q), _lib.strides(out), _lib.strides(kv),
            _lib.dtype_code(q), _lib.stream_handle(dev),
        )
    return out


def partial_prefill_attention_paged_varlen(
    query: torch.Tensor,
    kv_cache: torch.Tensor,
    block_tables: torch.Tensor,
    compute_positions: torch.Tensor,
    rows_per_request,
    blocks_per_request,
    scale: float | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Batched form of :func:`partial_prefill_attention_paged` for requests sharing one paged
    cache (one layer), in one launch per 16 requests.

    query: [sum(rows), num_q_heads, head_dim], the requests' rows back to back;
    compute_positions: [sum(rows)] int32, each row's position within its own request;
    block_tables: [num_requests, max_blocks] int32, request r using its first
    ``blocks_per_request[r]`` entries; rows_per_request / blocks_per_request: host integer
    sequences (the launch plan is built on the host, so the call never synchronises).
    Returns [sum(rows), num_q_heads, head_dim]. Extension with no reference counterpart (the
    reference runs one request per call); replaces a per-request loop over
    :func:`partial_prefill_attention_paged`.
    """
    dev = _lib.require_device(query, kv_cache, block_tables)
    rows = [int(r) for r in rows_per_request]
    blocks = [int(b) for b in blocks_per_request]
    if len(rows) != len(blocks):
        raise ValueError("rows_per_request and blocks_per_request differ in length")
    num_rows, num_q_heads, head_dim = query.shape
    nb_total, _, num_kv_heads, block_size, hd = kv_cache.shape
    if hd != head_dim:
        raise ValueError("query and kv_cache head_dim differ")
    if num_q_heads % num_kv_heads:
        raise ValueError("num_q_heads must be a multiple of num_kv_heads")
    if query.dtype != kv_cache.dtype:
        raise TypeError("query and kv_cache must share a dtype")
    if sum(rows) != num_rows:
        raise ValueError("rows_per_request must sum to the number of query rows")
    if block_tables.dim() != 2 or block_tables.shape[0] != len(rows):
        raise ValueError("block_tables must be [num_requests, max_blocks]")
    if any(b > block_tables.shape[1] for b in blocks):
        raise ValueError("a request has more blocks than its block-table row")
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    if out is None:
        out = torch.empty((num_rows, num_q_heads, head_dim), dtype=query.dtype, device=dev)
    if num_rows == 0:
        return out
    q = query if query.stride(-1) == 1 else query.contiguous()
    kv = kv_cache if kv_cache.stride(-1) == 1 else kv_cache.contiguous()
    pos = _lib.as_index(compute_positions, dev)
    if pos.shape[0] != num_rows:
        raise ValueError("compute_positions must have one entry per query row")
    bt = block_tables
    if bt.dtype != torch.int32 or bt.stride(1) != 1:
        bt = bt.to(torch.int32).contiguous()
    rows_a = _lib.i64_array(rows)
    blocks_a = _lib.i64_array(blocks)
    dt = _lib.dtype_code(q)
    ws_bytes = _lib.size_query("sb_partial_attention_paged_varlen_workspace_size", len(rows),
                               rows_a, blocks_a, num_q_heads, num_kv_heads, head_dim,
                               block_size, dt)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    with _lib.on_device(dev):
        _lib.call(
            "sb_partial_attention_paged_varlen",
            out.data_ptr(), q.data_ptr(), kv.data_ptr(), bt.data_ptr(), bt.stride(0),
            pos.data_ptr(), len(rows), rows_a, blocks_a, _lib.ptr(ws), ws_bytes, num_q_heads,
            num_kv_heads, head_dim, block_size, nb_total, float(scale), _lib.strides(q),
            _lib.strides(out), _lib.strides(kv), dt, _lib.stream_handle(dev),
        )
    return out


# ------------------------------------------------------------------------------------------
# Orchestrator
# ------------------------------------------------------------------------------------------

@dataclass
class PagedLayerResult:
    """Result of :func:`partial_prefill_layer_paged`: output [R, out_features] of the computed
    rows, their query [R, Hq, D] (rotated when RoPE was applied) and attention [R, Hq, D]."""

    output: torch.Tensor
    query: torch.Tensor
    attention: torch.Tensor


def partial_prefill_layer_paged(
    hidden_states: torch.Tensor,
    qkv_weight: torch.Tensor,
    output_projection: torch.Tensor,
    compute_positions: torch.Tensor,
    kv_cache: torch.Tensor,
    block_table: torch.Tensor,
    num_heads: int,
    num_kv_heads: int,
    head_dim: int,
    qkv_bias: torch.Tensor | None = None,
    output_bias: torch.Tensor | None = None,
    rope_base: float | None = None,
    scale: float | None = None,
    plan: PagedAttentionPlan | None = None,
) -> PagedLayerResult:
    """One attention layer of partial prefill, on the paged cache of that layer.

    The reference's single-layer orchestrator (semblend_core/triton_kernels.py:769-923)
    projects every row, runs MHA attention over a contiguous cache assembled per call and
    writes the new K/V into every layer. Here, per layer and for the computed rows only:
    (1) ``qkv_projection_paged`` — Q of the computed rows, their new K/V (RoPE at their
    positions when ``rope_base`` is given) written into this layer's paged cache, whose other
    slots already hold the scattered, RoPE-corrected donor K/V; (2) GQA attention of those
    rows over the cache (``partial_prefill_attention_paged``); (3) the output projection of
    the attention rows (torch's GEMM, fp32 accumulation, rounded to the input dtype). A model
    runs this once per layer with that layer's weights and cache; ``plan`` (from
    :func:`plan_partial_attention_paged` for these positions, made once per request) serves
    every layer's attention.
    """
    dev = _lib.require_device(hidden_states, qkv_weight, output_projection, kv_cache)
    q = qkv_projection_paged(hidden_states, qkv_weight, compute_positions, kv_cache,
                             block_table, num_heads, num_kv_heads, head_dim, qkv_bias=qkv_bias,
                             rope_base=rope_base)
    pos = _lib.as_index(compute_positions, dev)
    attn = partial_prefill_attention_paged(q, kv_cache, block_table, pos, scale=scale, plan=plan)
    flat = attn.reshape(attn.shape[0], num_heads * head_dim)
    out = torch.nn.functional.linear(flat, output_projection, output_bias)
    return PagedLayerResult(output=out, query=q, attention=attn)


@dataclass
class PartialPrefillResult:
    """Result of :func:`partial_prefill` (fields as semblend_core/triton_kernels.py:742-766).

    output: [seq_len, hidden] projected attention output (reuse rows zero);
    kv_cache: [num_layers, 2, num_heads, seq_len, head_dim] assembled target cache;
    positions_computed / positions_reused: compute-mask counts;
    computation_ratio: positions_computed / seq_len;
    *_time_ms: HIP-event timings of the scatter, projection and attention stages and of the
    whole call.
    """

    output: torch.Tensor
    kv_cache: torch.Tensor
    positions_computed: int
    positions_reused: int
    computation_ratio: float
    scatter_time_ms: float
    projection_time_ms: float
    attention_time_ms: float
    total_time_ms: float


def partial_prefill(
    hidden_states: torch.Tensor,
    donor_kv: torch.Tensor,
    qkv_weight: torch.Tensor,
    output_projection: torch.Tensor,
    donor_positions: torch.Tensor,
    target_positions: torch.Tensor,
    compute_mask: torch.Tensor,
    num_heads: int,
    head_dim: int,
    qkv_bias: torch.Tensor | None = None,
    output_bias: torch.Tensor | None = None,
    scale: float | None = None,
) -> PartialPrefillResult:
    """Single-layer partial prefill with donor KV reuse.

    Stages, with the reference's semantics (semblend_core/triton_kernels.py:769-923):
    (1) scatter donor K/V into a zeroed target cache [L, 2, H, S, D];
    (2) masked QKV projection (fp32, reuse rows zero);
    (3) merge: compute rows take the new K/V, reuse rows keep layer 0's scattered donor K/V;
    (4) partial attention over the merged layer-0 K/V in fp32, then the output projection,
        cast to the input dtype, with reuse rows zeroed;
    (5) the new K/V are written into the compute rows of EVERY layer of the target cache.
    Attention uses layer 0 only, as in the reference.
    """
    dev = _lib.require_device(hidden_states, donor_kv, qkv_weight, output_projection)
    seq_len = hidden_states.shape[0]
    num_layers = donor_kv.shape[0]
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    compute_mask = compute_mask.to(device=dev)
    if compute_mask.dtype != torch.bool:
        compute_mask = compute_mask != 0

    target_kv = torch.zeros((num_layers, 2, num_heads, seq_len, head_dim),
                            dtype=hidden_states.dtype, device=dev)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
    ev[0].record()
    scatter_donor_kv(target_kv, donor_kv, donor_positions, target_positions)
    ev[1].record()
    qkv_output = masked_qkv_projection(hidden_states, qkv_weight, compute_mask, qkv_bias)
    qkv = qkv_output.float().view(seq_len, 3, num_heads, head_dim)
    q_new = qkv[:, 0].permute(1, 0, 2)
    k_new = qkv[:, 1].permute(1, 0, 2)
    v_new = qkv[:, 2].permute(1, 0, 2)
    ev[2].record()

    cm = compute_mask.view(1, seq_len, 1)
    merged_k = torch.where(cm, k_new, target_kv[0, 0].float()).contiguous()
    merged_v = torch.where(cm, v_new, target_kv[0, 1].float()).contiguous()
    attn_output = partial_prefill_attention(q_new.contiguous(), merged_k, merged_v,
                                            compute_mask, scale)
    ev[3].record()

    attn_flat = attn_output.permute(1, 0, 2).reshape(seq_len, num_heads * head_dim)
    final_output = torch.nn.functional.linear(
        attn_flat,
        output_projection.float(),
        output_bias.float() if output_bias is not None else None,
    ).to(hidden_states.dtype)
    final_output = torch.where(compute_mask.view(seq_len, 1), final_output,
                               torch.zeros((), dtype=final_output.dtype, device=dev))

    # New K/V into the compute rows of every layer.
    sel = cm.unsqueeze(0)  # [1, 1, S, 1] against [L, H, S, D]
    new_k = k_new.to(target_kv.dtype).unsqueeze(0)
    new_v = v_new.to(target_kv.dtype).unsqueeze(0)
    target_kv[:, 0] = torch.where(sel, new_k, target_kv[:, 0])
    target_kv[:, 1] = torch.where(sel, new_v, target_kv[:, 1])
    ev[4].record()
    ev[4].synchronize()

    num_computed = int(compute_mask.sum().item())
    return PartialPrefillResult(
        output=final_output,
        kv_cache=target_kv,
        positions_computed=num_computed,
        positions_reused=seq_len - num_computed,
        computation_ratio=num_computed / seq_len if seq_len > 0 else 1.0,
        scatter_time_ms=ev[0].elapsed_time(ev[1]),
        projection_time_ms=ev[1].elapsed_time(ev[2]),
        attention_time_ms=ev[2].elapsed_time(ev[3]),
        total_time_ms=ev[0].elapsed_time(ev[4]),
    )
