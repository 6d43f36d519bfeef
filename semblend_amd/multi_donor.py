"""Multi-donor (composite) KV scatter on MI355X.

A composite plan fills one target sequence from several donors: every reused target position
names the donor that owns its KV and the position inside that donor
(``MultiDonorPositionMapping``, semblend_core/multi_donor_types.py:50-78; the per-position
``donor_map`` of ``build_multi_donor_attention_plan``, semblend_core/partial_attention.py:
306-435). The reference loads and scatters one donor at a time
(synapse_kv_connector/semblend_connector.py:1508-1701). Here one pass moves every pair of
every donor, all layers and heads, through a per-pair donor index and a per-donor table of
layer base addresses and strides (``sb_composite_scatter_paged_layers``), rotating K by
``target - donor`` as ``rope_correct_scatter_paged`` does.
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .partial_attention import PartialAttentionPlan, compute_donor_kv_indices
from .rope_correction import PreparedLaunch, inv_freq_table

__all__ = [
    "MultiDonorPositionMapping",
    "composite_pairs",
    "composite_pairs_from_plan",
    "composite_scatter_paged",
    "composite_scatter_paged_layers",
    "group_pairs_by_donor",
    "prepare_composite_scatter_paged_layers",
]


@dataclass(frozen=True)
class MultiDonorPositionMapping:
    """Donor-aware position mapping (semblend_core/multi_donor_types.py:50-78): entry i maps
    target position ``target_positions[i]`` to ``donor_positions[i]`` of donor
    ``donor_ids[i]``; RoPE correction rotates by ``target - donor`` per entry."""

    donor_ids: tuple[str, ...] = ()
    donor_positions: tuple[int, ...] = ()
    target_positions: tuple[int, ...] = ()

    @property
    def num_pairs(self) -> int:
        return len(self.target_positions)

    @property
    def needs_correction(self) -> bool:
        return any(d != t for d, t in zip(self.donor_positions, self.target_positions))

    def for_donor(self, donor_id: str) -> "MultiDonorPositionMapping":
        """The entries of one donor, in their original order."""
        keep = [i for i, did in enumerate(self.donor_ids) if did == donor_id]
        return MultiDonorPositionMapping(
            donor_ids=tuple(self.donor_ids[i] for i in keep),
            donor_positions=tuple(self.donor_positions[i] for i in keep),
            target_positions=tuple(self.target_positions[i] for i in keep),
        )


def composite_pairs(mapping: MultiDonorPositionMapping,
                    donor_order: Sequence[str] | None = None):
    """Flatten a mapping into the arrays the composite scatter takes.

    Returns ``(donor_order, donor_index, donor_positions, target_positions)``: the donors in
    the order their KV tensors must be passed (first appearance, unless ``donor_order`` is
    given) and int32 arrays with ``donor_index[i]`` indexing that order. Target positions
    must be distinct (each target has one owner); duplicates raise ``ValueError``, as do ids
    missing from ``donor_order``.
    """
    n = mapping.num_pairs
    if len(mapping.donor_ids) != n or len(mapping.donor_positions) != n:
        raise ValueError("donor_ids, donor_positions and target_positions differ in length")
    if donor_order is None:
        donor_order = tuple(dict.fromkeys(mapping.donor_ids))
    slot = {did: k for k, did in enumerate(donor_order)}
    missing = set(mapping.donor_ids) - slot.keys()
    if missing:
        raise ValueError(f"donor ids not in donor_order: {sorted(missing)}")
    tpos = np.asarray(mapping.target_positions, dtype=np.int64)
    if np.unique(tpos).size != tpos.size:
        raise ValueError("target positions must be distinct across donors")
    didx = np.fromiter((slot[d] for d in mapping.donor_ids), dtype=np.int32, count=n)
    return (tuple(donor_order), didx, np.asarray(mapping.donor_positions, dtype=np.int32),
            tpos.astype(np.int32))


def composite_pairs_from_plan(plan: PartialAttentionPlan, layer_idx: int = 0):
    """The reuse pairs of one layer of a multi-donor plan with each pair's owner taken from
    ``plan.donor_map`` (positions absent from it belong to ``plan.donor_id``, the primary
    donor; partial_attention.py:405-413)."""
    owner = dict(plan.donor_map)
    pairs = compute_donor_kv_indices(plan, layer_idx)
    return MultiDonorPositionMapping(
        donor_ids=tuple(owner.get(t, plan.donor_id) for _, t in pairs),
        donor_positions=tuple(d for d, _ in pairs),
        target_positions=tuple(t for _, t in pairs),
    )


def composite_scatter_paged_layers(
    kv_caches: list[torch.Tensor],
    donor_kvs: Sequence[Sequence[torch.Tensor]],
    block_table: torch.Tensor,
    donor_index,
    donor_positions,
    target_positions,
    rope: bool = True,
    rope_base: float = 10000.0,
    donor_first_positions: Sequence[int] | None = None,
    repeated_donor_rows: bool | None = None,
) -> list[torch.Tensor]:
    """Scatter pairs from several donors into every layer's paged cache in one pass.

    kv_caches: per layer ``[num_blocks, 2, H, block_size, D]``, one shape/stride/dtype.
    donor_kvs: per donor, per layer ``[2, H, S_k, D]`` (``donor_kvs[k][l]``); a donor's
        layers share shape and strides, donors may differ in length ``S_k`` and strides.
    donor_index / donor_positions / target_positions: per pair (int32 tensors or sequences).
    Pair i moves donor ``donor_index[i]``'s K and V at ``donor_positions[i]`` to
    ``target_positions[i]``; K is rotated by ``target - donor`` when ``rope``. Pairs whose
    donor index, donor position or target slot is out of range are skipped. Target positions
    must be distinct (the kernel does not order writes to one slot).
    donor_first_positions: per donor, the sequence position its tensors' row 0 holds
        (default 0): a tensor holding only a window ``[f, f + S_k)`` of a donor (one staged
        chunk) is read at ``donor_positions[i] - f`` and rotated by the true delta.
    repeated_donor_rows: whether one donor row may be the source of several pairs (the
        donors are then read through the caches); None decides from host positions and
        takes device positions as distinct. It changes speed, not results.
    """
    num_pairs = len(target_positions)
    if num_pairs == 0 or not kv_caches or not donor_kvs:
        return kv_caches
    num_layers = len(kv_caches)
    ref = kv_caches[0]
    nb_total, _, num_heads, block_size, head_dim = ref.shape
    dev = _lib.require_device(*kv_caches, *(t for per in donor_kvs for t in per))
    _check_same(kv_caches, "kv_caches")
    strides = _donor_strides(donor_kvs, ref, num_layers, donor_first_positions)
    if rope and head_dim % 2:
        raise ValueError("head_dim must be even for RoPE")
    kv_tab = _lib.address_table(kv_caches, dev)
    d_tab = _lib.address_table([t for per in donor_kvs for t in per], dev)
    bt = _lib.as_index(block_table, dev)
    didx = _lib.as_index(_as_tensor(donor_index), dev)
    dpos = _lib.as_index(_as_tensor(donor_positions), dev)
    tpos = _lib.as_index(_as_tensor(target_positions), dev)
    if not (didx.shape[0] == dpos.shape[0] == tpos.shape[0]):
        raise ValueError("donor_index, donor_positions and target_positions differ in length")
    if repeated_donor_rows is None:
        repeated_donor_rows = _lib.rows_repeat(donor_positions, donor_index)
    inv_freq = inv_freq_table(rope_base, head_dim, dev) if rope else None
    with _lib.on_device(dev):
        _lib.call(
            "sb_composite_scatter_paged_layers",
            kv_tab.data_ptr(), num_layers, d_tab.data_ptr(), len(donor_kvs),
            _lib.i64_array(strides), didx.data_ptr(), dpos.data_ptr(), tpos.data_ptr(),
            inv_freq.data_ptr() if inv_freq is not None else None, num_pairs, num_heads,
            block_size, head_dim, bt.data_ptr(), nb_total, bt.shape[0], _lib.strides(ref),
            _lib.dtype_code(ref), _lib.scatter_flags(repeated_donor_rows),
            _lib.stream_handle(dev),
        )
    return kv_caches


def composite_scatter_paged(
    kv_cache: torch.Tensor,
    donor_kvs: Mapping[str, torch.Tensor] | Sequence[torch.Tensor],
    block_table: torch.Tensor,
    mapping: MultiDonorPositionMapping,
    rope_base: float = 10000.0,
    rope: bool | None = None,
) -> torch.Tensor:
    """One layer from a ``MultiDonorPositionMapping``: ``donor_kvs`` maps donor id to its
    ``[2, H, S, D]`` KV (or is a sequence in the mapping's first-appearance order). RoPE is
    applied when ``rope`` is True, or, by default, when the mapping needs correction."""
    if mapping.num_pairs == 0:
        return kv_cache
    if isinstance(donor_kvs, Mapping):
        order, didx, dpos, tpos = composite_pairs(mapping, tuple(donor_kvs.keys()))
        tensors = [donor_kvs[d] for d in order]
    else:
        order, didx, dpos, tpos = composite_pairs(mapping)
        if len(donor_kvs) != len(order):
            raise ValueError(f"{len(order)} donors in the mapping, {len(donor_kvs)} tensors")
        tensors = list(donor_kvs)
    if rope is None:
        rope = mapping.needs_correction
    composite_scatter_paged_layers([kv_cache], [[t] for t in tensors], block_table, didx, dpos,
                                   tpos, rope=rope, rope_base=rope_base)
    return kv_cache


def _donor_strides(donor_kvs, ref: torch.Tensor, num_layers: int,
                   donor_first_positions) -> list[int]:
    """Per donor: kv, head and sequence strides (elements), rows held and first position, after
    checking every donor's layers against the caches (``num_layers`` layers like ``ref``)."""
    _, _, num_heads, _, head_dim = ref.shape
    if donor_first_positions is None:
        donor_first_positions = [0] * len(donor_kvs)
    if len(donor_first_positions) != len(donor_kvs):
        raise ValueError("one first position per donor")
    strides = []
    for k, per_layer in enumerate(donor_kvs):
        if len(per_layer) != num_layers:
            raise ValueError(f"donor {k} has {len(per_layer)} layers, the cache {num_layers}")
        _check_same(per_layer, f"donor {k} layers")
        d0 = per_layer[0]
        if d0.dim() != 4 or d0.shape[0] != 2 or d0.shape[1] != num_heads or d0.shape[3] != head_dim:
            raise ValueError(f"donor {k} must be [2, {num_heads}, S, {head_dim}]")
        if d0.dtype != ref.dtype:
            raise TypeError("donors and caches must share a dtype")
        if d0.stride(3) != 1:
            raise ValueError("donor head_dim must be contiguous (stride 1)")
        strides += [d0.stride(0), d0.stride(1), d0.stride(2), d0.shape[2],
                    int(donor_first_positions[k])]
    return strides


def group_pairs_by_donor(donor_index, donor_positions, target_positions, num_donors: int,
                         align: int = _lib.SB_GROUPED_PAIR_ALIGN, donors_per_launch: int = 16):
    """Host grouping of composite pairs for the grouped launch: pairs of an unknown donor
    are dropped (the indexed launch skips them), the rest are ordered by donor (stable), and
    every donor's run is padded with (-1, -1) pairs to a multiple of ``align``, except the last
    of each launch. Donors go in launches of ``donors_per_launch``.

    Returns one (first donor, donor count, int32 donor positions, int32 target positions,
    int64 segment ends) per launch that has pairs."""
    didx = np.asarray(donor_index, dtype=np.int64).reshape(-1)
    dpos = np.asarray(donor_positions, dtype=np.int64).reshape(-1)
    tpos = np.asarray(target_positions, dtype=np.int64).reshape(-1)
    if not (didx.size == dpos.size == tpos.size):
        raise ValueError("donor_index, donor_positions and target_positions differ in length")
    keep = (didx >= 0) & (didx < num_donors)
    didx, dpos, tpos = didx[keep], dpos[keep], tpos[keep]
    order = np.argsort(didx, kind="stable")
    didx, dpos, tpos = didx[order], dpos[order], tpos[order]
    bounds = np.searchsorted(didx, np.arange(num_donors + 1))
    launches = []
    for first in range(0, num_donors, donors_per_launch):
        count = min(donors_per_launch, num_donors - first)
        parts_d, parts_t, ends, n = [], [], [], 0
        for k in range(first, first + count):
            seg_d = dpos[bounds[k]:bounds[k + 1]]
            seg_t = tpos[bounds[k]:bounds[k + 1]]
            last = k == first + count - 1
            pad = 0 if last else (-len(seg_d)) % align
            parts_d += [seg_d, np.full(pad, -1)]
            parts_t += [seg_t, np.full(pad, -1)]
            n += len(seg_d) + pad
            ends.append(n)
        if bounds[first + count] > bounds[first]:
            launches.append((first, count, np.concatenate(parts_d).astype(np.int32),
                             np.concatenate(parts_t).astype(np.int32),
                             np.asarray(ends, dtype=np.int64)))
    return launches


def prepare_composite_scatter_paged_layers(
    kv_caches: list[torch.Tensor],
    donor_kvs: Sequence[Sequence[torch.Tensor]],
    block_table: torch.Tensor,
    donor_index,
    donor_positions,
    target_positions,
    rope: bool = True,
    rope_base: float = 10000.0,
    donor_first_positions: Sequence[int] | None = None,
    repeated_donor_rows: bool | None = None,
) -> PreparedLaunch | None:
    """Bind :func:`composite_scatter_paged_layers` once, with the pairs grouped by donor on the
    host (device tensors are read back once), so that each workgroup's pairs share one donor
    (``sb_composite_scatter_paged_layers_grouped``: the donor's strides and layer table are
    read once per workgroup, not per pair). Calling the returned object enqueues the launches
    (one per 16 donors) on the current stream; it holds the uploaded pairs and tables, so the
    tensors must keep their storage. Same results as the per-call form. Returns None when no
    pair names a known donor."""
    if not kv_caches or not donor_kvs:
        return None
    num_layers = len(kv_caches)
    ref = kv_caches[0]
    nb_total, _, num_heads, block_size, head_dim = ref.shape
    dev = _lib.require_device(*kv_caches, *(t for per in donor_kvs for t in per))
    _check_same(kv_caches, "kv_caches")
    strides = _donor_strides(donor_kvs, ref, num_layers, donor_first_positions)
    if rope and head_dim % 2:
        raise ValueError("head_dim must be even for RoPE")
    host = [x.cpu() if isinstance(x, torch.Tensor) else x
            for x in (donor_index, donor_positions, target_positions)]
    if repeated_donor_rows is None:
        repeated_donor_rows = _lib.rows_repeat(_as_tensor(host[1]), _as_tensor(host[0]))
    launches = group_pairs_by_donor(*host, num_donors=len(donor_kvs))
    if not launches:
        return None
    kv_tab = _lib.address_table(kv_caches, dev)
    bt = _lib.as_index(block_table, dev)
    inv_freq = inv_freq_table(rope_base, head_dim, dev) if rope else None
    keep = [kv_tab, bt, inv_freq]
    calls = []
    for first, count, dp, tp, ends in launches:
        d_tab = _lib.address_table([t for per in donor_kvs[first:first + count] for t in per],
                                   dev)
        both = _lib.upload_index(torch.from_numpy(np.concatenate([dp, tp])), dev)
        n = int(dp.size)
        st = _lib.i64_array(strides[5 * first:5 * (first + count)])
        en = _lib.i64_array(ends.tolist())
        keep += [d_tab, both, st, en]
        calls.append(("sb_composite_scatter_paged_layers_grouped", (
            kv_tab.data_ptr(), num_layers, d_tab.data_ptr(), count, st, en, both.data_ptr(),
            both.data_ptr() + 4 * n, inv_freq.data_ptr() if inv_freq is not None else None, n,
            num_heads, block_size, head_dim, bt.data_ptr(), nb_total, bt.shape[0],
            _lib.strides(ref), _lib.dtype_code(ref), _lib.scatter_flags(repeated_donor_rows))))
    return PreparedLaunch(calls[0][0], calls[0][1], tuple(keep), dev, more=tuple(calls[1:]))


def _as_tensor(x) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        return x
    return torch.as_tensor(np.asarray(x, dtype=np.int32))


def _check_same(ts: Sequence[torch.Tensor], name: str) -> None:
    t0 = ts[0]
    for t in ts:
        if t.shape != t0.shape or t.stride() != t0.stride() or t.dtype != t0.dtype:
            raise ValueError(f"all {name} must share shape, strides and dtype")
        if t.data_ptr() % 16:
            raise ValueError(f"{name} base addresses must be 16-byte aligned")
