"""Partial-attention plans — drop-in for ``semblend_core.partial_attention``
(semblend_core/partial_attention.py).

Host-side data structures that tell the kernels which target positions reuse donor K/V
(REUSE, with a donor position) and which need fresh Q/K/V (PARTIAL / FULL), per layer. The
kernels consume two products of a plan: the boolean compute mask
(:func:`compute_attention_mask`) and the (donor_pos, target_pos) copy pairs
(:func:`compute_donor_kv_indices`).

The types, enum values, field names and builder semantics are those of the reference,
including two of its behaviours that callers can observe:

* ``build_attention_plan`` only recognises ``"copy_from_donor"`` and ``"placeholder"`` slot
  actions; other actions (e.g. ``"recompute"``) add no position mask, while the plan's
  counts come from the ``copy_positions`` / ``placeholder_positions`` arguments
  (semblend_core/partial_attention.py:134-156, :200-201).
* ``build_multi_donor_attention_plan`` treats ``"recompute"`` as the compute action and
  ignores ``"placeholder"`` (:332-357).
"""

from __future__ import annotations

from collections import Counter
from dataclasses import dataclass, field
from enum import Enum

import numpy as np

__all__ = [
    "AttentionMode",
    "LayerMask",
    "PartialAttentionPlan",
    "PositionMask",
    "build_attention_plan",
    "build_multi_donor_attention_plan",
    "compute_attention_mask",
    "compute_donor_kv_indices",
]


class AttentionMode(Enum):
    """How one position (or layer) is computed (semblend_core/partial_attention.py:28-42)."""

    FULL = "full"              # fresh Q/K/V, ordinary prefill
    REUSE = "reuse"            # donor K/V reused, nothing computed
    PARTIAL = "partial"        # fresh Q/K/V attending over all cached K/V
    SKIP_LAYER = "skip_layer"  # layer skipped altogether


@dataclass(frozen=True)
class PositionMask:
    """Mode of one target position; ``donor_pos`` is set for REUSE positions."""

    target_pos: int
    mode: AttentionMode
    donor_pos: int | None = None


@dataclass(frozen=True)
class LayerMask:
    """Per-layer strategy: whole-layer recompute, or per-position masks."""

    layer_idx: int
    recompute_all: bool
    deviation_score: float
    position_masks: list[PositionMask] = field(default_factory=list)
    verification_source: str = "bathtub"


@dataclass(frozen=True)
class PartialAttentionPlan:
    """Per-layer, per-position plan (fields as semblend_core/partial_attention.py:73-102).

    ``computation_ratio`` is the fraction of per-position projection work relative to a full
    prefill; ``donor_map`` maps target positions to donor ids for multi-donor plans.
    """

    target_len: int
    donor_len: int
    donor_id: str
    layer_masks: list[LayerMask]
    num_reuse_positions: int
    num_partial_positions: int
    num_full_layers: int
    computation_ratio: float
    donor_map: tuple[tuple[int, str], ...] = ()


def _slot_target(action: dict) -> int:
    return action.get("targetPos", action.get("target_pos", 0))


def _slot_donor(action: dict):
    return action.get("donorPos", action.get("donor_pos"))


def _layer_hint(layer_hints: list[dict] | None, layer_idx: int) -> tuple[bool, float]:
    """(recompute_all, deviation_score) for a layer; camelCase or snake_case keys."""
    if not layer_hints or layer_idx >= len(layer_hints):
        return False, 0.0
    hint = layer_hints[layer_idx]
    return (
        hint.get("recomputeAll", hint.get("recompute_all", False)),
        hint.get("deviationScore", hint.get("deviation_score", 0.0)),
    )


def _layer_masks(position_masks: list[PositionMask], target_len: int,
                 layer_hints: list[dict] | None, num_layers: int) -> tuple[list[LayerMask], int]:
    """Expand shared position masks into per-layer masks; FULL masks for recompute layers."""
    layers: list[LayerMask] = []
    full = 0
    for idx in range(num_layers):
        recompute_all, score = _layer_hint(layer_hints, idx)
        if recompute_all:
            full += 1
            masks = [PositionMask(target_pos=i, mode=AttentionMode.FULL)
                     for i in range(target_len)]
            layers.append(LayerMask(layer_idx=idx, recompute_all=True, deviation_score=score,
                                    position_masks=masks))
        else:
            layers.append(LayerMask(layer_idx=idx, recompute_all=False, deviation_score=score,
                                    position_masks=list(position_masks)))
    return layers, full


def _computation_ratio(num_layers: int, target_len: int, num_full: int,
                       num_partial: int) -> float:
    """(partial layers x partial positions + full layers x all positions) / (layers x len)."""
    if num_layers <= 0 or target_len <= 0:
        return 1.0
    work = (num_layers - num_full) * num_partial + num_full * target_len
    return work / (num_layers * target_len)


def build_attention_plan(
    donor_id: str,
    target_len: int,
    donor_len: int,
    copy_positions: list[int],
    placeholder_positions: list[int],
    slot_actions: list[dict],
    layer_hints: list[dict] | None = None,
    num_layers: int = 32,
) -> PartialAttentionPlan:
    """Plan from a transfer plan's slot actions (semblend_core/partial_attention.py:105-230).

    ``copy_from_donor`` actions become REUSE masks carrying their donor position;
    ``placeholder`` actions become PARTIAL masks. Layers whose hint sets ``recomputeAll``
    get FULL masks for every position.
    """
    position_masks: list[PositionMask] = []
    for action in slot_actions:
        kind = action.get("action", "")
        if kind == "copy_from_donor":
            position_masks.append(PositionMask(_slot_target(action), AttentionMode.REUSE,
                                               _slot_donor(action)))
        elif kind == "placeholder":
            position_masks.append(PositionMask(_slot_target(action), AttentionMode.PARTIAL))
    layers, num_full = _layer_masks(position_masks, target_len, layer_hints, num_layers)
    num_partial = len(placeholder_positions)
    return PartialAttentionPlan(
        target_len=target_len,
        donor_len=donor_len,
        donor_id=donor_id,
        layer_masks=layers,
        num_reuse_positions=len(copy_positions),
        num_partial_positions=num_partial,
        num_full_layers=num_full,
        computation_ratio=_computation_ratio(num_layers, target_len, num_full, num_partial),
    )


def compute_attention_mask(plan: PartialAttentionPlan, layer_idx: int) -> np.ndarray:
    """bool[target_len]: True where the layer computes Q/K/V (PARTIAL or FULL).

    Layers beyond the plan, and recompute-all layers, are all True
    (semblend_core/partial_attention.py:233-270).
    """
    if layer_idx >= len(plan.layer_masks) or plan.layer_masks[layer_idx].recompute_all:
        return np.ones(plan.target_len, dtype=bool)
    mask = np.zeros(plan.target_len, dtype=bool)
    for pm in plan.layer_masks[layer_idx].position_masks:
        if pm.mode in (AttentionMode.PARTIAL, AttentionMode.FULL) and pm.target_pos < plan.target_len:
            mask[pm.target_pos] = True
    return mask


def compute_donor_kv_indices(plan: PartialAttentionPlan, layer_idx: int) -> list[tuple[int, int]]:
    """(donor_pos, target_pos) for the layer's REUSE positions, in mask order.

    Empty for layers beyond the plan and for recompute-all layers
    (semblend_core/partial_attention.py:273-303).
    """
    if layer_idx >= len(plan.layer_masks) or plan.layer_masks[layer_idx].recompute_all:
        return []
    return [
        (pm.donor_pos, pm.target_pos)
        for pm in plan.layer_masks[layer_idx].position_masks
        if pm.mode == AttentionMode.REUSE and pm.donor_pos is not None
    ]


def build_multi_donor_attention_plan(
    target_len: int,
    slot_actions: list[dict],
    layer_hints: list[dict] | None = None,
    num_layers: int = 32,
) -> PartialAttentionPlan:
    """Plan from multi-donor slot actions (semblend_core/partial_attention.py:306-435).

    ``copy_from_donor`` -> REUSE (and ``donor_map[target] = donorId`` when given);
    ``recompute`` -> PARTIAL. ``donor_len`` is one past the largest donor position of any
    action; ``donor_id`` is the most frequent donor in ``donor_map`` ("" if none).
    """
    position_masks: list[PositionMask] = []
    donor_map: dict[int, str] = {}
    num_copy = 0
    num_recompute = 0
    for action in slot_actions:
        kind = action.get("action", "")
        tpos = _slot_target(action)
        if kind == "copy_from_donor":
            position_masks.append(PositionMask(tpos, AttentionMode.REUSE, _slot_donor(action)))
            num_copy += 1
            did = action.get("donorId", action.get("donor_id"))
            if did:
                donor_map[tpos] = did
        elif kind == "recompute":
            position_masks.append(PositionMask(tpos, AttentionMode.PARTIAL))
            num_recompute += 1
    layers, num_full = _layer_masks(position_masks, target_len, layer_hints, num_layers)

    donor_positions = [d for d in (_slot_donor(a) for a in slot_actions) if d is not None]
    donor_len = max((d + 1 for d in donor_positions), default=0)
    donor_len = max(donor_len, 0)
    primary = Counter(donor_map.values()).most_common(1)[0][0] if donor_map else ""
    return PartialAttentionPlan(
        target_len=target_len,
        donor_len=donor_len,
        donor_id=primary,
        layer_masks=layers,
        num_reuse_positions=num_copy,
        num_partial_positions=num_recompute,
        num_full_layers=num_full,
        computation_ratio=_computation_ratio(num_layers, target_len, num_full, num_recompute),
        donor_map=tuple(donor_map.items()),
    )
