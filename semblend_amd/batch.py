"""Multi-request KV reuse over a shared paged cache (a serving batch).

The reference corrects and attends one request at a time: its connectors walk each request's
layers and call the per-layer functions (synapse_kv_connector/model_runner_hook.py:519-585,
semblend/integration/trtllm/pytorch_backend.py:106-154). :class:`KVReuseBatch` holds the
requests of one batch and runs

* :meth:`KVReuseBatch.scatter_rope` — donor K/V into the paged cache with K rotated by
  ``target - donor`` (``rope_correct_scatter_paged`` semantics), or copied unrotated with
  ``rope=False`` (``scatter_donor_kv_paged``), for every layer: one launch per request, each
  covering all of that request's layers and pairs;
* :meth:`KVReuseBatch.attention` — the recompute rows of every request attending causally
  over their own context in one layer's cache: one launch for up to 16 requests.

Every call is asynchronous on torch's current stream; the batch layout (padded block-table
matrix, row offsets) is built once on the host from the requests' sizes, so no call
synchronises.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch

from . import _lib
from .rope_correction import prepare_scatter_paged_layers
from .triton_kernels import partial_prefill_attention_paged_varlen


@dataclass
class ReuseRequest:
    """One request of a batch.

    block_table: [num_blocks] int32, the request's logical blocks in the shared pool;
    donor_kvs: one donor buffer [2, num_kv_heads, donor_len, head_dim] per layer;
    donor_positions / target_positions: [P] int32 reuse pairs (donor row -> target position);
    compute_positions: [R] int32 recompute positions (ascending is fastest).
    """

    block_table: torch.Tensor
    donor_kvs: Sequence[torch.Tensor]
    donor_positions: torch.Tensor
    target_positions: torch.Tensor
    compute_positions: torch.Tensor


class KVReuseBatch:
    """Requests sharing per-layer paged caches ``kv_caches`` ([num_blocks, 2, num_kv_heads,
    block_size, head_dim] each, one per layer)."""

    def __init__(self, kv_caches: Sequence[torch.Tensor], requests: Sequence[ReuseRequest],
                 rope_base: float = 10000.0):
        if not kv_caches:
            raise ValueError("kv_caches is empty")
        self.kv_caches = list(kv_caches)
        self.requests = list(requests)
        self.rope_base = float(rope_base)
        dev = _lib.require_device(*self.kv_caches)
        for r in self.requests:
            if len(r.donor_kvs) != len(self.kv_caches):
                raise ValueError("every request needs one donor buffer per layer")
            if r.donor_positions.shape[0] != r.target_positions.shape[0]:
                raise ValueError("donor_positions and target_positions differ in length")
        self.device = dev
        self.rows_per_request = [int(r.compute_positions.shape[0]) for r in self.requests]
        self.blocks_per_request = [int(r.block_table.shape[0]) for r in self.requests]
        max_blocks = max(self.blocks_per_request, default=0)
        tables = torch.full((len(self.requests), max(max_blocks, 1)), -1, dtype=torch.int32,
                            device=dev)
        for i, r in enumerate(self.requests):
            tables[i, : self.blocks_per_request[i]] = _lib.as_index(r.block_table, dev)
        self.block_tables = tables
        if self.requests:
            self.compute_positions = torch.cat(
                [_lib.as_index(r.compute_positions, dev) for r in self.requests])
        else:
            self.compute_positions = torch.zeros(0, dtype=torch.int32, device=dev)
        self._scatter_calls: dict[bool, list] = {}
        self.row_offsets = [0]
        for n in self.rows_per_request:
            self.row_offsets.append(self.row_offsets[-1] + n)

    @property
    def num_rows(self) -> int:
        return self.row_offsets[-1]

    def scatter_rope(self, rope: bool = True) -> None:
        """Donor K/V of every request into every layer's cache (K rotated when ``rope``).

        The per-request launches are validated and bound on first use (one
        ``PreparedScatter`` each), so a repeated step costs one C call per request."""
        calls = self._scatter_calls.get(rope)
        if calls is None:
            calls = [prepare_scatter_paged_layers(
                         self.kv_caches, list(r.donor_kvs), r.block_table, r.donor_positions,
                         r.target_positions, self.rope_base if rope else None)
                     for r in self.requests]
            calls = [c for c in calls if c is not None]
            self._scatter_calls[rope] = calls
        for call in calls:
            call()

    def attention(self, layer: int, query: torch.Tensor, scale: float | None = None,
                  out: torch.Tensor | None = None) -> torch.Tensor:
        """Attention of every request's recompute rows over ``kv_caches[layer]``.

        query: [num_rows, num_q_heads, head_dim], the requests' rows back to back in request
        order (request i's rows at ``row_offsets[i]:row_offsets[i + 1]``)."""
        return partial_prefill_attention_paged_varlen(
            query, self.kv_caches[layer], self.block_tables, self.compute_positions,
            self.rows_per_request, self.blocks_per_request, scale=scale, out=out)
