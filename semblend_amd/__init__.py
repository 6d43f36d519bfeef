"""semblend_amd — SemBlend's KV-reuse kernel path on AMD Instinct MI355X (gfx950).

Drop-in modules (same call surface as SemBlend's ``semblend_core`` modules):

* :mod:`semblend_amd.triton_kernels`   — donor-KV scatter, masked projection, partial
  attention, single-layer orchestrator;
* :mod:`semblend_amd.rope_correction`  — RoPE delta / NoPE correction of donor K;
* :mod:`semblend_amd.partial_attention` — plan types and mask / pair builders;
* :mod:`semblend_amd.pipeline`         — ``PositionMapping``.

Extensions: :mod:`semblend_amd.batch` (several requests over one paged pool) and
:mod:`semblend_amd.multi_donor` (composite scatter from several donors in one pass).

The compute runs in hand-written HIP kernels (``libsemblend_hip.so``, C ABI in
``include/semblend_hip.h``) on torch's current stream. ``semblend_amd.compat.install()``
aliases the modules under the ``semblend_core`` / ``synapse_kv_connector`` import paths.
"""

from . import _lib
from .partial_attention import (
    AttentionMode,
    LayerMask,
    PartialAttentionPlan,
    PositionMask,
    build_attention_plan,
    build_multi_donor_attention_plan,
    compute_attention_mask,
    compute_donor_kv_indices,
)
from .pipeline import PositionMapping

__version__ = "0.1.0"
HAS_HIP = _lib.available()

__all__ = [
    "AttentionMode",
    "HAS_HIP",
    "LayerMask",
    "PartialAttentionPlan",
    "PositionMapping",
    "PositionMask",
    "build_attention_plan",
    "build_multi_donor_attention_plan",
    "compute_attention_mask",
    "compute_donor_kv_indices",
]
