"""RoPE delta correction of reused donor K on MI355X — drop-in for
``semblend_core.rope_correction`` (semblend_core/rope_correction.py).

Same function names, parameters, defaults, return values and in-place conventions as the
reference module. Every function runs hand-written HIP kernels from ``libsemblend_hip.so``
through its C ABI on torch's current stream; CPU tensors are rejected.

Convention (semblend_core/rope_correction.py:163-178, :317-326): interleaved (GPT-J) pairs
``(2i, 2i+1)`` rotated by ``theta = delta * inv_freq[i]`` with
``inv_freq[i] = 1 / base ** (2i / head_dim)``:

    e' = e * cos(theta) - o * sin(theta)
    o' = e * sin(theta) + o * cos(theta)

computed in fp32 and rounded once to the cache dtype (the reference's CPU path, :328; its
Triton kernels store fp16 regardless of the cache dtype, :183-190, which is not reproduced).
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib

# Kept for import compatibility with callers that re-export it
# (synapse_kv_connector/rope_correction.py:8-21). There is no Triton here; the kernels are
# HIP and their availability is HAS_HIP.
HAS_TRITON = False
HAS_HIP = _lib.available()

__all__ = [
    "HAS_TRITON",
    "HAS_HIP",
    "apply_rope_delta_inplace",
    "apply_rope_deltas_inplace_layers",
    "inv_freq_table",
    "nope_permute_paged_kv",
    "nope_permute_paged_kv_layers",
    "paged_layout",
    "permute_paged_kv_with_rope",
    "permute_paged_kv_with_rope_layers",
    "prepare_permute_paged_kv_layers",
    "standard_view",
    "rope_correct_k",
    "rope_correct_k_inplace",
    "rope_correct_scatter_paged",
    "rope_correct_scatter_paged_layers",
]

_INV_FREQ_CACHE: dict[tuple[float, int, torch.device], torch.Tensor] = {}


def inv_freq_table(rope_base: float, head_dim: int, device: torch.device) -> torch.Tensor:
    """fp32 ``1 / base ** (arange(0, D, 2) / D)`` on ``device``, cached.

    The table is evaluated with the reference's exact torch expression
    (semblend_core/rope_correction.py:234-238) on the host and copied once to the device, so
    the angles ``delta * inv_freq`` are bit-identical to the reference's: at |delta| ~ 4096 a
    one-ulp difference in inv_freq would move the angle by ~5e-4 rad.
    """
    key = (float(rope_base), int(head_dim), torch.device(device))
    tab = _INV_FREQ_CACHE.get(key)
    if tab is None:
        host = 1.0 / (rope_base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
        tab = host.to(device)
        _INV_FREQ_CACHE[key] = tab
    return tab


def _check_head_dim(head_dim: int, actual: int, fn: str) -> None:
    if head_dim != actual:
        raise ValueError(
            f"{fn}: head_dim={head_dim} does not match the tensor's last dimension {actual}"
        )
    if head_dim % 2:
        raise ValueError(f"{fn}: head_dim must be even for RoPE, got {head_dim}")


def rope_correct_scatter_paged(
    kv_cache: torch.Tensor,
    donor_kv: torch.Tensor,
    block_table: torch.Tensor,
    donor_positions: torch.Tensor,
    target_positions: torch.Tensor,
    rope_base: float = 10000.0,
    head_dim: int | None = None,
) -> torch.Tensor:
    """Scatter donor KV into a paged cache, rotating K by ``target - donor``; V is copied.

    kv_cache: [num_blocks, 2, num_heads, block_size, head_dim] (any strides);
    donor_kv: [2, num_heads, donor_seq_len, head_dim]; block_table: [num_blocks_per_seq].
    Returns kv_cache (modified in place). Pairs whose donor position, logical block or
    physical block is out of range are skipped.
    Reference: semblend_core/rope_correction.py:193-282.
    """
    num_pairs = len(donor_positions)
    if len(target_positions) != num_pairs:
        raise ValueError(f"donor_positions ({num_pairs}) and target_positions "
                         f"({len(target_positions)}) differ in length")
    if num_pairs == 0:
        return kv_cache
    nb_total, _, num_heads, block_size, hd = kv_cache.shape
    head_dim = hd if head_dim is None else head_dim
    _check_head_dim(head_dim, hd, "rope_correct_scatter_paged")
    dev = _lib.require_device(kv_cache, donor_kv)
    if donor_kv.dtype != kv_cache.dtype:
        raise TypeError("donor_kv and kv_cache must share a dtype")
    bt = _lib.as_index(block_table, dev)
    dpos = _lib.as_index(donor_positions, dev)
    tpos = _lib.as_index(target_positions, dev)
    inv_freq = inv_freq_table(rope_base, head_dim, dev)
    with _lib.on_device(dev):
        _lib.call(
            "sb_rope_correct_scatter_paged",
            kv_cache.data_ptr(), donor_kv.data_ptr(), bt.data_ptr(), dpos.data_ptr(),
            tpos.data_ptr(), inv_freq.data_ptr(), num_pairs, num_heads, block_size, head_dim,
            donor_kv.shape[2], nb_total, bt.shape[0], _lib.strides(kv_cache),
            _lib.strides(donor_kv), _lib.dtype_code(kv_cache), _lib.stream_handle(dev),
        )
    return kv_cache


def rope_correct_scatter_paged_layers(
    kv_caches: list[torch.Tensor],
    donor_kvs: list[torch.Tensor],
    block_table: torch.Tensor,
    donor_positions: torch.Tensor,
    target_positions: torch.Tensor,
    rope_base: float = 10000.0,
    repeated_donor_rows: bool | None = None,
) -> list[torch.Tensor]:
    """``rope_correct_scatter_paged`` over many layers in one launch.

    kv_caches / donor_kvs: one tensor per layer, all with the same shape, strides and dtype.
    cos/sin of each pair are evaluated once and reused for every layer and head.
    repeated_donor_rows: as in ``prepare_scatter_paged_layers``, except that None takes
    device positions as distinct (no synchronisation per call). Extension
    with no reference counterpart; it replaces a per-layer loop around
    ``rope_correct_scatter_paged`` (semblend/integration/trtllm/pytorch_backend.py:106-154).
    """
    if repeated_donor_rows is None:
        repeated_donor_rows = _lib.rows_repeat(donor_positions)
    call = prepare_scatter_paged_layers(kv_caches, donor_kvs, block_table, donor_positions,
                                        target_positions, rope_base, repeated_donor_rows)
    if call is not None:
        call()
    return kv_caches


class PreparedLaunch:
    """Validated launches of the library bound to their tensors' addresses; calling the object
    enqueues them on torch's current stream. It holds the device tables, index tensors and
    workspaces they read, so those live as long as it does."""

    def __init__(self, entry: str, args: tuple, keep: tuple, device: torch.device,
                 more: tuple = ()):
        self.launches = [(entry, args)] + list(more)
        self.entry, self.args, self.keep, self.device = entry, args, keep, device

    def __call__(self) -> None:
        with _lib.on_device(self.device):
            st = _lib.stream_handle(self.device)
            for entry, args in self.launches:
                _lib.call(entry, *args, st)


# The multi-layer scatter's prepared form (kept under its first name).
PreparedScatter = PreparedLaunch


def prepare_scatter_paged_layers(
    kv_caches: list[torch.Tensor],
    donor_kvs: list[torch.Tensor],
    block_table: torch.Tensor,
    donor_positions: torch.Tensor,
    target_positions: torch.Tensor,
    rope_base: float | None = 10000.0,
    repeated_donor_rows: bool | None = None,
) -> PreparedScatter | None:
    """Check the inputs of the multi-layer paged scatter once and bind them: K is rotated by
    ``target - donor`` with RoPE base ``rope_base``, or copied unrotated (with V) when
    ``rope_base`` is None. Returns None when there are no pairs. For callers that repeat the
    same scatter every step: the host work of validation, address tables and index uploads
    is done here, not per launch; the tensors must keep their storage afterwards.

    repeated_donor_rows: whether a donor position may be the source of several pairs (e.g.
    chunks whose deltas make their donor windows overlap). The launch then reads donors
    through the caches, which serves the repeats from L2 / Infinity Cache; otherwise it reads
    them with nontemporal loads, faster when each donor row is read once. None finds out
    from the positions (one device-to-host read for device positions, here only; under HIP
    graph capture device positions count as distinct). Results are the same either way."""
    if len(kv_caches) != len(donor_kvs):
        raise ValueError("kv_caches and donor_kvs must have the same length")
    num_pairs = len(donor_positions)
    if len(target_positions) != num_pairs:
        raise ValueError("donor_positions and target_positions differ in length")
    if num_pairs == 0 or not kv_caches:
        return None
    ref, dref = kv_caches[0], donor_kvs[0]
    nb_total, _, num_heads, block_size, head_dim = ref.shape
    rope = rope_base is not None
    if rope:
        _check_head_dim(head_dim, head_dim, "rope_correct_scatter_paged_layers")
    dev = _lib.require_device(*kv_caches, *donor_kvs)
    _check_uniform(kv_caches, "kv_caches")
    _check_uniform(donor_kvs, "donor_kvs")
    if dref.dtype != ref.dtype:
        raise TypeError("donor_kvs and kv_caches must share a dtype")
    if repeated_donor_rows is None:
        # one device-to-host read for device positions, except under graph capture
        repeated_donor_rows = _lib.rows_repeat(
            donor_positions, sync=not torch.cuda.is_current_stream_capturing())
    kv_tab = _layer_table(kv_caches, dev)
    d_tab = _layer_table(donor_kvs, dev)
    bt = _lib.as_index(block_table, dev)
    dpos = _lib.as_index(donor_positions, dev)
    tpos = _lib.as_index(target_positions, dev)
    tail = (num_pairs, num_heads, block_size, head_dim, dref.shape[2], nb_total, bt.shape[0],
            _lib.strides(ref), _lib.strides(dref), _lib.dtype_code(ref),
            _lib.scatter_flags(repeated_donor_rows))
    head = (kv_tab.data_ptr(), d_tab.data_ptr(), len(kv_caches), bt.data_ptr(),
            dpos.data_ptr(), tpos.data_ptr())
    if rope:
        inv_freq = inv_freq_table(float(rope_base), head_dim, dev)
        return PreparedScatter("sb_rope_correct_scatter_paged_layers",
                               head + (inv_freq.data_ptr(),) + tail,
                               (kv_tab, d_tab, bt, dpos, tpos, inv_freq), dev)
    return PreparedScatter("sb_scatter_donor_kv_paged_layers", head + tail,
                           (kv_tab, d_tab, bt, dpos, tpos), dev)


def _check_uniform(ts: list[torch.Tensor], name: str) -> None:
    t0 = ts[0]
    for t in ts[1:]:
        if t.shape != t0.shape or t.stride() != t0.stride() or t.dtype != t0.dtype:
            raise ValueError(f"all {name} must share shape, strides and dtype")
    for t in ts:
        if t.data_ptr() % 16:
            raise ValueError(f"{name} base addresses must be 16-byte aligned")


def _layer_table(ts: list[torch.Tensor], dev: torch.device) -> torch.Tensor:
    return _lib.address_table(ts, dev)


def _rope_k(out: torch.Tensor, k: torch.Tensor, dpos, tpos, head_dim, rope_base) -> None:
    dev = _lib.require_device(k, out)
    if k.dim() == 3:
        k4, o4 = k.unsqueeze(0), out.unsqueeze(0)
    elif k.dim() == 4:
        k4, o4 = k, out
    else:
        raise ValueError("k_tensor must be [H, S, D] or [L, H, S, D]")
    num_layers, num_heads, seq_len, hd = k4.shape
    _check_head_dim(head_dim, hd, "rope_correct_k")
    d = _lib.as_index(dpos, dev)
    t = _lib.as_index(tpos, dev)
    if d.shape[0] != t.shape[0]:
        raise ValueError("donor_positions and target_positions differ in length")
    inv_freq = inv_freq_table(rope_base, head_dim, dev)
    ws = torch.empty(2 * seq_len, dtype=torch.int32, device=dev)
    with _lib.on_device(dev):
        _lib.call(
            "sb_rope_correct_k",
            o4.data_ptr(), k4.data_ptr(), d.data_ptr(), t.data_ptr(), inv_freq.data_ptr(),
            ws.data_ptr(), d.shape[0], num_layers, num_heads, seq_len, head_dim,
            _lib.strides(o4), _lib.strides(k4), _lib.dtype_code(k4), _lib.stream_handle(dev),
        )


def rope_correct_k(
    k_tensor: torch.Tensor,
    donor_positions: torch.Tensor,
    target_positions: torch.Tensor,
    head_dim: int = 128,
    rope_base: float = 10000.0,
) -> torch.Tensor:
    """Return a copy of ``k_tensor`` whose rows at the donor positions are rotated.

    k_tensor: [num_heads, seq_len, head_dim] or [num_layers, num_heads, seq_len, head_dim].
    For each pair i (in order) the row at ``donor_positions[i]`` is rotated by
    ``target_positions[i] - donor_positions[i]`` and rounded to the tensor dtype; a row named
    by several pairs is rotated once per pair. The input is not modified.
    Reference: semblend_core/rope_correction.py:336-399.
    """
    _lib.require_device(k_tensor)
    out = torch.empty_like(k_tensor)
    if k_tensor.stride(-1) != 1:
        k_tensor = k_tensor.contiguous()
    if out.stride(-1) != 1:
        out = torch.empty_like(k_tensor, memory_format=torch.contiguous_format)
    _rope_k(out, k_tensor, donor_positions, target_positions, head_dim, rope_base)
    return out


def rope_correct_k_inplace(
    k_tensor: torch.Tensor,
    donor_positions: torch.Tensor,
    target_positions: torch.Tensor,
    head_dim: int = 128,
    rope_base: float = 10000.0,
    distinct_donors: bool = False,
) -> torch.Tensor:
    """In-place form of :func:`rope_correct_k` (same result, written back into k_tensor).

    Only rows named by a pair are read and written. ``distinct_donors=True`` is the caller's
    guarantee that no donor position repeats (e.g. a whole-sequence correction with
    d = 0..S-1): the rows are then rotated pair by pair in one launch, without building the
    per-position index that orders repeated rotations (a repeated position would race).
    Extension with no reference counterpart.
    """
    _lib.require_device(k_tensor)
    if distinct_donors and k_tensor.stride(-1) == 1:
        dev = k_tensor.device
        if k_tensor.dim() == 3:
            k4 = k_tensor.unsqueeze(0)
        elif k_tensor.dim() == 4:
            k4 = k_tensor
        else:
            raise ValueError("k_tensor must be [H, S, D] or [L, H, S, D]")
        num_layers, num_heads, seq_len, hd = k4.shape
        _check_head_dim(head_dim, hd, "rope_correct_k_inplace")
        d = _lib.as_index(donor_positions, dev)
        t = _lib.as_index(target_positions, dev)
        if d.shape[0] != t.shape[0]:
            raise ValueError("donor_positions and target_positions differ in length")
        if d.shape[0] == 0:
            return k_tensor
        inv_freq = inv_freq_table(rope_base, head_dim, dev)
        with _lib.on_device(dev):
            _lib.call(
                "sb_rope_correct_k_distinct",
                k4.data_ptr(), d.data_ptr(), t.data_ptr(), inv_freq.data_ptr(), d.shape[0],
                num_layers, num_heads, seq_len, head_dim, _lib.strides(k4),
                _lib.dtype_code(k4), _lib.stream_handle(dev),
            )
        return k_tensor
    if k_tensor.stride(-1) != 1:
        work = k_tensor.contiguous()
        _rope_k(work, work, donor_positions, target_positions, head_dim, rope_base)
        k_tensor.copy_(work)
        return k_tensor
    _rope_k(k_tensor, k_tensor, donor_positions, target_positions, head_dim, rope_base)
    return k_tensor


def permute_paged_kv_with_rope(
    kv_cache: torch.Tensor,
    block_table: torch.Tensor,
    permutation: list[tuple[int, int]],
    rope_base: float = 10000.0,
) -> None:
    """Move (source, target) logical positions inside a paged cache, rotating K by
    ``target - source``; V is copied.

    Every source row is read before any target row is written (the reference snapshots all
    sources first, semblend_core/rope_correction.py:437-448), so overlapping permutations
    such as swaps are exact. kv_cache layout: [num_blocks, 2, num_heads, block_size, head_dim].
    Reference: semblend_core/rope_correction.py:407-476.
    """
    if not permutation:
        return
    dev = _lib.require_device(kv_cache)
    nb_total, _, num_heads, block_size, head_dim = kv_cache.shape
    _check_head_dim(head_dim, head_dim, "permute_paged_kv_with_rope")
    src, tgt = _pairs_on_device(permutation, dev)
    bt = _lib.as_index(block_table, dev)
    inv_freq = inv_freq_table(rope_base, head_dim, dev)
    ws = torch.empty((len(permutation), 2, num_heads, head_dim), dtype=kv_cache.dtype,
                     device=dev)
    with _lib.on_device(dev):
        _lib.call(
            "sb_permute_paged_kv_with_rope",
            kv_cache.data_ptr(), bt.data_ptr(), src.data_ptr(), tgt.data_ptr(),
            inv_freq.data_ptr(), ws.data_ptr(), len(permutation), num_heads, block_size,
            head_dim, nb_total, bt.shape[0], _lib.strides(kv_cache), _lib.dtype_code(kv_cache),
            _lib.stream_handle(dev),
        )


def _sequential_v_moves(permutation: list[tuple[int, int]]) -> list[tuple[int, int]]:
    """Resolve a sequence of in-place copies ``V[t] = V[s]`` (done in list order) into
    (original source, target) pairs, one per distinct target, with the same final contents.

    The reference copies V rows one pair at a time (semblend_core/rope_correction.py:650-653),
    so a later pair reads what an earlier pair wrote. Tracking, for every written position,
    which original row it now holds reproduces that outcome with a single snapshot-and-write
    pass. Positions are logical; distinct logical blocks are assumed to map to distinct
    physical blocks, as in engine block tables.
    """
    holds: dict[int, int] = {}
    for s, t in permutation:
        holds[t] = holds.get(s, s)
    return list(holds.items())


def nope_permute_paged_kv(
    kv_cache: torch.Tensor,
    block_table: torch.Tensor,
    permutation: list[tuple[int, int]],
    rope_base: float = 10000.0,
) -> None:
    """NoPE two-step correction: ``K[tgt] = R(tgt) R(-src) K[src]``; V copied.

    K rows are read before any K row is written; V rows follow the reference's sequential
    copy semantics (see ``_sequential_v_moves``). Both rotations run in fp32 with one
    rounding to the cache dtype.
    Reference: semblend_core/rope_correction.py:599-697 (CPU path :786-823).
    """
    if not permutation:
        return
    dev = _lib.require_device(kv_cache)
    nb_total, _, num_heads, block_size, head_dim = kv_cache.shape
    _check_head_dim(head_dim, head_dim, "nope_permute_paged_kv")
    src, tgt = _pairs_on_device(permutation, dev)
    vmoves = _sequential_v_moves(permutation)
    # holds maps target -> original source; emit (source, target) pairs.
    vsrc, vtgt = _pairs_on_device([(s_, t_) for t_, s_ in vmoves], dev)
    bt = _lib.as_index(block_table, dev)
    inv_freq = inv_freq_table(rope_base, head_dim, dev)
    ws = torch.empty((len(permutation) + len(vmoves), num_heads, head_dim),
                     dtype=kv_cache.dtype, device=dev)
    with _lib.on_device(dev):
        _lib.call(
            "sb_nope_permute_paged_kv",
            kv_cache.data_ptr(), bt.data_ptr(), src.data_ptr(), tgt.data_ptr(),
            len(permutation), vsrc.data_ptr(), vtgt.data_ptr(), len(vmoves),
            inv_freq.data_ptr(), ws.data_ptr(), num_heads, block_size, head_dim, nb_total,
            bt.shape[0], _lib.strides(kv_cache), _lib.dtype_code(kv_cache),
            _lib.stream_handle(dev),
        )


def _rotation_counts(positions: list[int], block_size: int,
                     num_blocks_per_seq: int) -> tuple[dict[int, int], int]:
    """Host-side resolution of ``apply_rope_delta_inplace``'s position list.

    Returns ({logical position: times it is rotated}, positions processed). Positions whose
    logical block lies past the table are skipped; negative positions index blocks from the
    end of the table, as ``block_table[pos // block_size]`` does in Python
    (semblend_core/rope_correction.py:758-763); below -num_blocks_per_seq blocks that raises
    IndexError there and here.
    """
    counts: dict[int, int] = {}
    processed = 0
    for pos in positions:
        blk_idx = pos // block_size
        if blk_idx >= num_blocks_per_seq:
            continue
        if blk_idx < -num_blocks_per_seq:
            raise IndexError(
                f"position {pos} indexes block {blk_idx} of a {num_blocks_per_seq}-entry table")
        if blk_idx < 0:
            blk_idx += num_blocks_per_seq
        logical = blk_idx * block_size + pos % block_size
        counts[logical] = counts.get(logical, 0) + 1
        processed += 1
    return counts, processed


def apply_rope_delta_inplace(
    kv_cache: torch.Tensor,
    block_table: torch.Tensor,
    positions: list[int],
    delta: int,
    rope_base: float = 10000.0,
) -> int:
    """Rotate K at the given logical positions by ``delta`` in place; V untouched.

    Accepts the vLLM flash-attn layout [2, num_blocks, block_size, num_kv_heads, head_dim]
    and the standard [num_blocks, 2, num_heads, block_size, head_dim], detected exactly as
    the reference does (semblend_core/rope_correction.py:740). Positions whose logical block
    lies beyond the block table are skipped; a position listed k times is rotated k times.
    Returns the number of positions processed (duplicates counted), or 0 for delta == 0 or
    an empty list. Reference: semblend_core/rope_correction.py:699-783.
    """
    if delta == 0 or not positions:
        return 0
    if not -_lib.MAX_ROPE_DELTA < int(delta) < _lib.MAX_ROPE_DELTA:
        raise ValueError(f"apply_rope_delta_inplace: |delta| must be below 2^31, got {delta} "
                         "(the kernels' sin/cos reduce angles below 2^32 exactly)")
    dev = _lib.require_device(kv_cache)
    shape, st = kv_cache.shape, kv_cache.stride()
    # The K plane starts at the tensor's own address in both layouts (kv index 0); strides
    # (block, head, pos, dim) are read off the full tensor, so no view is made.
    if kv_cache.ndim == 5 and shape[0] == 2 and shape[1] != 2:  # vLLM [2, NB, bs, H, D]
        nb_total, block_size, num_heads, head_dim = shape[1], shape[2], shape[3], shape[4]
        kst = (st[1], st[3], st[2], st[4])
    else:                                                        # [NB, 2, H, bs, D]
        nb_total, num_heads, block_size, head_dim = shape[0], shape[2], shape[3], shape[4]
        kst = (st[0], st[2], st[3], st[4])
    _check_head_dim(head_dim, head_dim, "apply_rope_delta_inplace")
    nbs = block_table.shape[0]
    counts, modified = _rotation_counts(positions, block_size, nbs)
    if not counts:
        return 0
    bt = _lib.as_index(block_table, dev)
    inv_freq = inv_freq_table(rope_base, head_dim, dev)
    reps = list(counts.values())
    repeated = any(c != 1 for c in reps)
    keys = list(counts.keys())
    with _lib.on_device(dev):
        inline = _lib.SB_INLINE_POSITIONS_MAX
        if len(keys) <= inline or torch.cuda.is_current_stream_capturing():
            # Short lists (and any list under graph capture, in launches of up to 256
            # positions) travel inside the launch: no index upload.
            for c0 in range(0, len(keys), inline):
                _lib.call(
                    "sb_apply_rope_delta_inplace_host",
                    kv_cache.data_ptr(), bt.data_ptr(), _lib.i32_array(keys[c0:c0 + inline]),
                    _lib.i32_array(reps[c0:c0 + inline]) if repeated else None,
                    len(keys[c0:c0 + inline]), int(delta), inv_freq.data_ptr(), num_heads,
                    block_size, head_dim, nb_total, nbs, _lib.i64_array(kst),
                    _lib.dtype_code(kv_cache), _lib.stream_handle(dev),
                )
            return modified
        pos_t = _lib.upload_index(torch.tensor(keys, dtype=torch.int32), dev)
        rep_t = _lib.upload_index(torch.tensor(reps, dtype=torch.int32), dev) if repeated else None
        _lib.call(
            "sb_apply_rope_delta_inplace",
            kv_cache.data_ptr(), bt.data_ptr(), pos_t.data_ptr(),
            None if rep_t is None else rep_t.data_ptr(), len(counts), int(delta),
            inv_freq.data_ptr(), num_heads, block_size, head_dim, nb_total, nbs,
            _lib.i64_array(kst), _lib.dtype_code(kv_cache), _lib.stream_handle(dev),
        )
    return modified


def _delta_rounds(positions, deltas, block_size: int,
                  num_blocks_per_seq: int) -> tuple[list[tuple[np.ndarray, np.ndarray]], int]:
    """Host-side resolution of ``apply_rope_deltas_inplace_layers``' (position, delta) list,
    with the rule of ``apply_rope_delta_inplace`` applied to each entry as a one-position call
    (semblend_core/rope_correction.py:732-783): delta 0 and positions whose logical block lies
    past the table are skipped; negative positions index blocks from the end of the table
    (below -num_blocks_per_seq blocks: IndexError, as there).

    Returns (rounds, entries processed). Round r holds the r-th occurrence of every logical
    position, in list order, as (int32 positions, int32 deltas): within a round the positions
    are distinct, and a position's rotations land in list order across the rounds."""
    pos = np.asarray(positions, dtype=np.int64).reshape(-1)
    dlt = np.asarray(deltas, dtype=np.int64).reshape(-1)
    if pos.shape != dlt.shape:
        raise ValueError(f"positions ({pos.size}) and deltas ({dlt.size}) differ in length")
    if np.any(np.abs(dlt) >= _lib.MAX_ROPE_DELTA):
        raise ValueError("apply_rope_deltas_inplace_layers: every |delta| must be below 2^31 "
                         "(the kernels' sin/cos reduce angles below 2^32 exactly)")
    blk = pos // block_size                      # floor division, as Python's //
    keep = (dlt != 0) & (blk < num_blocks_per_seq)
    if np.any(keep & (blk < -num_blocks_per_seq)):
        bad = int(pos[keep & (blk < -num_blocks_per_seq)][0])
        raise IndexError(f"position {bad} indexes block {bad // block_size} of a "
                         f"{num_blocks_per_seq}-entry table")
    logical = np.where(blk < 0, blk + num_blocks_per_seq, blk) * block_size + pos % block_size
    logical, dlt = logical[keep], dlt[keep]
    n = int(logical.size)
    if n == 0:
        return [], 0
    order = np.argsort(logical, kind="stable")
    srt = logical[order]
    start = np.r_[0, np.flatnonzero(np.diff(srt)) + 1]
    first = np.repeat(start, np.diff(np.r_[start, n]))
    occurrence = np.empty(n, dtype=np.int64)
    occurrence[order] = np.arange(n) - first
    rounds = []
    for r in range(int(occurrence.max()) + 1):
        sel = occurrence == r
        rounds.append((logical[sel].astype(np.int32), dlt[sel].astype(np.int32)))
    return rounds, n


def apply_rope_deltas_inplace_layers(
    kv_caches: list[torch.Tensor],
    block_table: torch.Tensor,
    positions,
    deltas,
    rope_base: float = 10000.0,
    layout: str | None = None,
) -> int:
    """Rotate K in place at many positions, each by its own delta, in every layer's cache,
    with one launch per occurrence round (one launch when no position repeats); V untouched.

    Same result as, and the same count returned by, ::

        sum(apply_rope_delta_inplace(kv, block_table, [p], d, rope_base)
            for kv in kv_caches for p, d in zip(positions, deltas))

    i.e. the per-(layer, pair) loop of the TRT-LLM post-load hook
    (semblend/integration/trtllm/semblend_provider.py:305-318) or, for the per-delta caller
    pattern, one ``apply_rope_delta_inplace`` call per distinct delta over its positions: a
    position listed several times is rotated that many times, in list order, rounded to the
    cache dtype after each rotation. Entries with delta 0 or past the block table count as
    not processed.

    kv_caches: one cache per layer, all with one shape, strides and dtype, in ``layout``
    ("standard" [NB, 2, H, bs, D], "vllm" [2, NB, bs, H, D], "trt" [NB, 2, tpb, H, D]; None:
    the reference's detection rule); positions, deltas: integer sequences (or tensors, read on
    the host) of one length; every |delta| < 2^31. Extension with no single-call reference
    counterpart (it replaces the loops above).
    """
    if not kv_caches:
        return 0
    dev = _lib.require_device(*kv_caches)
    _check_uniform(kv_caches, "kv_caches")
    nb, heads, bs, hd, st = paged_layout(kv_caches[0], layout)
    _check_head_dim(hd, hd, "apply_rope_deltas_inplace_layers")
    if st[4] != 1:
        raise ValueError("head_dim must be contiguous (stride 1)")
    if isinstance(positions, torch.Tensor):
        positions = positions.cpu()
    if isinstance(deltas, torch.Tensor):
        deltas = deltas.cpu()
    nbs = block_table.shape[0]
    rounds, processed = _delta_rounds(positions, deltas, bs, nbs)
    if not rounds:
        return 0
    bt = _lib.as_index(block_table, dev)
    inv = inv_freq_table(rope_base, hd, dev)
    tab = _lib.address_table(kv_caches, dev)
    kst = _lib.i64_array((st[0], st[2], st[3], st[4]))
    inline = _lib.SB_INLINE_POSITIONS_MAX
    capturing = torch.cuda.is_current_stream_capturing()
    with _lib.on_device(dev):
        stream = _lib.stream_handle(dev)
        for pos_r, dlt_r in rounds:
            n = int(pos_r.size)
            if n <= inline or capturing:
                # in the launch's arguments, up to 256 positions per launch
                for c0 in range(0, n, inline):
                    p_c, d_c = pos_r[c0:c0 + inline], dlt_r[c0:c0 + inline]
                    _lib.call(
                        "sb_apply_rope_deltas_inplace_layers_host",
                        tab.data_ptr(), len(kv_caches), bt.data_ptr(),
                        p_c.ctypes.data_as(_lib.I32P), d_c.ctypes.data_as(_lib.I32P),
                        int(p_c.size), inv.data_ptr(), heads, bs, hd, nb, nbs, kst,
                        _lib.dtype_code(kv_caches[0]), stream,
                    )
                continue
            # one upload of [positions | deltas] per round
            both = _lib.upload_index(torch.from_numpy(np.concatenate([pos_r, dlt_r])), dev)
            _lib.call(
                "sb_apply_rope_deltas_inplace_layers",
                tab.data_ptr(), len(kv_caches), bt.data_ptr(), both.data_ptr(),
                both.data_ptr() + 4 * n, n, inv.data_ptr(), heads, bs, hd, nb, nbs, kst,
                _lib.dtype_code(kv_caches[0]), stream,
            )
    return processed * len(kv_caches)


# ------------------------------------------------------------------------------------------
# Engine cache layouts and the multi-layer permutations
# ------------------------------------------------------------------------------------------

_LAYOUT_AXES = {
    # layout -> axes of (block, kv, head, pos, dim) in the tensor's own dimension order
    "standard": (0, 1, 2, 3, 4),   # [NB, 2, H, bs, D]
    "vllm": (1, 0, 3, 2, 4),       # [2, NB, bs, H, D]   (vLLM flash-attn)
    "trt": (0, 1, 3, 2, 4),        # [NB, 2, tpb, H, D]  (TensorRT-LLM)
}


def _resolve_layout(kv_cache: torch.Tensor, layout: str | None) -> str:
    if layout is None:
        # the reference's detection rule (semblend_core/rope_correction.py:740); TRT-LLM
        # caches cannot be told from standard ones by shape and need layout="trt"
        vllm = kv_cache.dim() == 5 and kv_cache.shape[0] == 2 and kv_cache.shape[1] != 2
        return "vllm" if vllm else "standard"
    if layout not in _LAYOUT_AXES:
        raise ValueError(f"layout must be one of {sorted(_LAYOUT_AXES)}, got {layout!r}")
    return layout


def standard_view(kv_cache: torch.Tensor, layout: str | None = None) -> torch.Tensor:
    """The cache as a [num_blocks, 2, num_heads, block_size, head_dim] view (no copy), from the
    standard, vLLM flash-attn [2, NB, bs, H, D] or TRT-LLM [NB, 2, tpb, H, D] layout. Every
    entry point of this package that takes a paged cache addresses it through its strides,
    so the view is what they take."""
    if kv_cache.dim() != 5:
        raise ValueError("a paged cache is 5-dimensional")
    return kv_cache.permute(*_LAYOUT_AXES[_resolve_layout(kv_cache, layout)])


def paged_layout(kv_cache: torch.Tensor, layout: str | None = None):
    """(num_blocks, num_heads, block_size, head_dim, element strides in (block, kv, head, pos,
    dim) order) of a paged cache in the given layout (None: the reference's detection rule)."""
    v = standard_view(kv_cache, layout)
    if v.shape[1] != 2:
        raise ValueError(f"no K/V axis of size 2 in a {layout or 'standard'} cache of shape "
                         f"{tuple(kv_cache.shape)}")
    nb, _, h, bs, d = v.shape
    return nb, h, bs, d, tuple(v.stride())


def _pairs_on_device(permutation, dev: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """(sources, targets) int32 device tensors from a list of (src, tgt) pairs or a [P, 2]
    tensor, uploaded once from pinned memory without blocking the host."""
    if isinstance(permutation, torch.Tensor):
        pairs = permutation.reshape(-1, 2).to(torch.int32)
    else:
        pairs = torch.tensor([(int(a), int(b)) for a, b in permutation],
                             dtype=torch.int32).reshape(-1, 2)
    if pairs.device.type == "cpu":
        pairs = _lib.pinned_upload(pairs.contiguous(), dev)
    else:
        pairs = pairs.to(dev)
    pairs = pairs.t().contiguous()
    return pairs[0], pairs[1]


def prepare_permute_paged_kv_layers(
    kv_caches: list[torch.Tensor],
    block_table: torch.Tensor,
    permutation,
    rope_base: float = 10000.0,
    nope: bool = False,
    layout: str | None = None,
    max_workspace_bytes: int = 1 << 30,
) -> PreparedLaunch | None:
    """Validate and bind the permutation of every layer's cache (``permute_paged_kv_with_rope``
    semantics, or ``nope_permute_paged_kv`` with ``nope=True``) once: the pairs are uploaded
    once, the layer table and the snapshot workspace are built once, and calling the returned
    object enqueues one snapshot launch and one write launch per group of layers (all layers
    in one group while the snapshot fits ``max_workspace_bytes``). Each call applies the
    permutation again (it is not idempotent). Returns None for an empty permutation.

    kv_caches: one cache per layer, all in ``layout`` ("standard" [NB, 2, H, bs, D], "vllm"
    [2, NB, bs, H, D], "trt" [NB, 2, tpb, H, D]; None: the reference's detection rule) with
    the same shape, strides and dtype; block_table: [num_blocks_per_seq]; permutation: list of
    (source, target) logical positions, or a [P, 2] integer tensor.
    Replaces the per-layer loop of synapse_kv_connector/model_runner_hook.py:519-585.
    """
    if not kv_caches or len(permutation) == 0:
        return None
    dev = _lib.require_device(*kv_caches)
    _check_uniform(kv_caches, "kv_caches")
    nb, heads, bs, hd, st = paged_layout(kv_caches[0], layout)
    _check_head_dim(hd, hd, "prepare_permute_paged_kv_layers")
    if st[4] != 1:
        raise ValueError("head_dim must be contiguous (stride 1)")
    src, tgt = _pairs_on_device(permutation, dev)
    num_pairs = int(src.shape[0])
    bt = _lib.as_index(block_table, dev)
    inv = inv_freq_table(rope_base, hd, dev)
    es = kv_caches[0].element_size()
    keep = [src, tgt, bt, inv]
    if nope:
        if isinstance(permutation, torch.Tensor):
            permutation = [tuple(p) for p in permutation.reshape(-1, 2).tolist()]
        vmoves = _sequential_v_moves(list(permutation))
        vsrc, vtgt = _pairs_on_device([(s_, t_) for t_, s_ in vmoves], dev)
        keep += [vsrc, vtgt]
        per_layer = (num_pairs + len(vmoves)) * heads * hd * es
    else:
        per_layer = num_pairs * 2 * heads * hd * es
    group = max(1, min(len(kv_caches), max_workspace_bytes // max(per_layer, 1)))
    ws = torch.empty(group * per_layer, dtype=torch.uint8, device=dev)
    keep.append(ws)
    strides = _lib.i64_array(st)
    keep.append(strides)
    launches = []
    for g0 in range(0, len(kv_caches), group):
        layers = kv_caches[g0:g0 + group]
        tab = _lib.address_table(layers, dev)
        keep.append(tab)
        if nope:
            args = (tab.data_ptr(), len(layers), bt.data_ptr(), src.data_ptr(), tgt.data_ptr(),
                    num_pairs, vsrc.data_ptr(), vtgt.data_ptr(), int(vsrc.shape[0]),
                    inv.data_ptr(), ws.data_ptr(), heads, bs, hd, nb, bt.shape[0], strides,
                    _lib.dtype_code(kv_caches[0]))
            launches.append(("sb_nope_permute_paged_kv_layers", args))
        else:
            args = (tab.data_ptr(), len(layers), bt.data_ptr(), src.data_ptr(), tgt.data_ptr(),
                    inv.data_ptr(), ws.data_ptr(), num_pairs, heads, bs, hd, nb, bt.shape[0],
                    strides, _lib.dtype_code(kv_caches[0]))
            launches.append(("sb_permute_paged_kv_with_rope_layers", args))
    return PreparedLaunch(launches[0][0], launches[0][1], tuple(keep), dev,
                          more=tuple(launches[1:]))


def permute_paged_kv_with_rope_layers(
    kv_caches: list[torch.Tensor],
    block_table: torch.Tensor,
    permutation,
    rope_base: float = 10000.0,
    layout: str | None = None,
) -> None:
    """``permute_paged_kv_with_rope`` applied to every layer's cache in one launch pair, in the
    standard, vLLM flash-attn or TRT-LLM layout (addressed through strides, so the vLLM
    caches the reference mis-decodes at rope_correction.py:432 are corrected exactly).
    Extension with no reference counterpart; replaces the per-layer loop of
    synapse_kv_connector/model_runner_hook.py:519-585. See
    :func:`prepare_permute_paged_kv_layers` to bind once and launch per step."""
    call = prepare_permute_paged_kv_layers(kv_caches, block_table, permutation, rope_base,
                                           nope=False, layout=layout)
    if call is not None:
        call()


def nope_permute_paged_kv_layers(
    kv_caches: list[torch.Tensor],
    block_table: torch.Tensor,
    permutation,
    rope_base: float = 10000.0,
    layout: str | None = None,
) -> None:
    """``nope_permute_paged_kv`` (K: R(tgt) R(-src); V: the reference's sequential copies) on
    every layer's cache in one set of launches, in any of the three layouts. Extension with no
    reference counterpart; replaces the NoPE branch of the per-layer loop at
    synapse_kv_connector/model_runner_hook.py:543-551."""
    call = prepare_permute_paged_kv_layers(kv_caches, block_table, permutation, rope_base,
                                           nope=True, layout=layout)
    if call is not None:
        call()
