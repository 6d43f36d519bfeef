"""Position-pair carrier consumed by the RoPE correction path.

Only ``PositionMapping`` is on the KV-reuse path: the donor-discovery pipeline that fills it
(embedding search, alignment) runs elsewhere. Reference: semblend_core/pipeline.py:62-81.
"""

from __future__ import annotations

from dataclasses import dataclass, field

__all__ = ["PositionMapping"]


@dataclass
class PositionMapping:
    """Pairs ``(donor_positions[i], target_positions[i])``: the KV at the donor position is
    placed at the target position, K rotated by ``target - donor``."""

    donor_positions: list[int] = field(default_factory=list)
    target_positions: list[int] = field(default_factory=list)

    @property
    def num_pairs(self) -> int:
        return len(self.donor_positions)

    @property
    def needs_correction(self) -> bool:
        """True when at least one pair moves (donor != target)."""
        return any(d != t for d, t in zip(self.donor_positions, self.target_positions))
