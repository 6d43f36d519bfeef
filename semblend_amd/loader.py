"""Chunked donor-KV load from host memory, overlapped with RoPE correction on MI355X.

In the reference, LMCache copies the donor's 256-token KV chunks from host memory into the
paged cache (synapse_kv_connector/semblend_connector.py:465-498; chunk alignment :1197-1222)
and the RoPE correction runs afterwards, in place, as a separate pass over the cache
(``_apply_rope_after_load``). Here the two are one streamed pass: each chunk is copied
host-to-device into a small ring of staging slots, and, as soon as it has
landed, rotated and scattered from the slot straight into every layer's paged cache while
the next chunk is still on the PCIe link. The slot is read as a donor window that starts at
the chunk's first position (``sb_composite_scatter_paged_layers`` with that first position),
so rows are found at ``d - c * T`` and K is rotated by the true ``t - d``. The cache is
written once; no pass reads it back.

Host chunks use LMCache's ``KV_2LTD`` layout: ``[2, num_layers, T, H * D]`` (or the same
memory as ``[2, L, T, H, D]``), in pinned memory so the copies are asynchronous.
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np
import torch

from . import _lib
from .rope_correction import inv_freq_table

__all__ = ["ChunkedKVLoader", "group_pairs_by_chunk"]


def group_pairs_by_chunk(donor_positions, target_positions, chunk_tokens: int,
                         num_chunks: int):
    """Pairs sorted by the donor chunk that holds them (stable, so pairs keep their order
    within a chunk): an int32 ``[3, P]`` array of (donor position, target position, 0 — the
    donor index the composite entry takes) and ``offsets[c]:offsets[c + 1]``, chunk c's
    run. Pairs whose donor position lies outside the chunks are dropped."""
    d = np.asarray(donor_positions, dtype=np.int64).reshape(-1)
    t = np.asarray(target_positions, dtype=np.int64).reshape(-1)
    if d.shape != t.shape:
        raise ValueError("donor_positions and target_positions differ in length")
    c = np.where(d >= 0, d // chunk_tokens, -1)
    keep = (c >= 0) & (c < num_chunks)
    d, t, c = d[keep], t[keep], c[keep]
    order = np.argsort(c, kind="stable")
    c = c[order]
    arr = np.stack([d[order], t[order], np.zeros_like(d)]).astype(np.int32)
    offsets = np.searchsorted(c, np.arange(num_chunks + 1), side="left")
    return arr, offsets


class ChunkedKVLoader:
    """Streams donor KV chunks into paged caches with RoPE correction on the fly.

    kv_caches: per layer ``[num_blocks, 2, H, block_size, D]`` (one shape, strides, dtype).
    block_table: the target sequence's block table.
    chunk_tokens: tokens per host chunk (LMCache: 256); the last chunk may be shorter.
    slots: staging buffers in the ring, allocated once, here (8 x 14.7 MB for Qwen2.5-7B's
        28 layers x 4 KV heads x 128 at 256 tokens).

    Schedule: the host-to-device copies are enqueued on torch's current stream and the
    scatters on the loader's own stream (default priority). Copy c waits for the scatter that
    last read its slot, the scatter waits for copy c, and the current stream finally waits for
    the last scatter, so work queued after ``load`` sees the caches. (The opposite assignment,
    copies on a side stream behind a wait on a still-pending event, made the copy enqueue
    block the host until the event completed and left the link idle between chunks.)

    ``load`` may be called repeatedly (e.g. once per donor of a composite plan); the ring
    and its events carry over, so consecutive loads also overlap.
    """

    def __init__(self, kv_caches: list[torch.Tensor], block_table: torch.Tensor,
                 chunk_tokens: int = 256, slots: int = 8, rope_base: float = 10000.0):
        if not kv_caches:
            raise ValueError("kv_caches is empty")
        if chunk_tokens <= 0 or slots <= 0:
            raise ValueError("chunk_tokens and slots must be positive")
        self.dev = _lib.require_device(*kv_caches)
        ref = kv_caches[0]
        for t in kv_caches:
            if t.shape != ref.shape or t.stride() != ref.stride() or t.dtype != ref.dtype:
                raise ValueError("all kv_caches must share shape, strides and dtype")
            if t.data_ptr() % 16:
                raise ValueError("kv_caches base addresses must be 16-byte aligned")
        if ref.stride(4) != 1:
            raise ValueError("head_dim must be contiguous (stride 1)")
        self.kv_caches = list(kv_caches)
        self.nb_total, _, self.num_heads, self.block_size, self.head_dim = ref.shape
        self.num_layers = len(kv_caches)
        self.dtype = ref.dtype
        self.chunk_tokens = int(chunk_tokens)
        self.rope_base = float(rope_base)
        self.block_table = _lib.as_index(block_table, self.dev)
        self._kv_tab = _lib.address_table(self.kv_caches, self.dev)
        self._kv_strides = _lib.strides(ref)
        self._dtype_code = _lib.dtype_code(ref)
        self._inv_freq = inv_freq_table(self.rope_base, self.head_dim, self.dev)
        shape = (2, self.num_layers, self.chunk_tokens, self.num_heads, self.head_dim)
        self._slots = [torch.empty(shape, dtype=self.dtype, device=self.dev)
                       for _ in range(slots)]
        # per slot: device table of the layer windows of a full chunk
        self._slot_tabs = [self._layer_table(s, self.chunk_tokens) for s in self._slots]
        self.scatter_stream = torch.cuda.Stream(device=self.dev)
        self._loaded = [torch.cuda.Event() for _ in range(slots)]
        self._free = [torch.cuda.Event() for _ in range(slots)]
        self._next = 0

    def _window(self, slot: torch.Tensor, tc: int) -> torch.Tensor:
        """The first tc tokens of a slot as a contiguous [2, L, tc, H, D] tensor."""
        n = 2 * self.num_layers * tc * self.num_heads * self.head_dim
        return slot.view(-1)[:n].view(2, self.num_layers, tc, self.num_heads, self.head_dim)

    def _layer_table(self, slot: torch.Tensor, tc: int) -> torch.Tensor:
        w = self._window(slot, tc)
        return _lib.address_table([w[:, l] for l in range(self.num_layers)], self.dev)

    def _group(self, donor_positions, target_positions, num_chunks: int):
        """``group_pairs_by_chunk`` with the pair array uploaded (one asynchronous copy
        from pinned memory on the current stream)."""
        arr, offsets = group_pairs_by_chunk(donor_positions, target_positions,
                                            self.chunk_tokens, num_chunks)
        return _lib.pinned_upload(torch.from_numpy(arr), self.dev), offsets

    def load(self, chunks: Sequence[torch.Tensor], donor_positions, target_positions,
             rope: bool = True) -> None:
        """Load one donor's chunks and scatter its pairs.

        chunks: host tensors, chunk c holding donor tokens ``[c * T, c * T + T_c)``.
        donor_positions / target_positions: host integer sequences of the pairs (donor
            positions in the donor's full sequence). K is rotated by ``target - donor``
            when ``rope``. Chunks that no pair reads are not copied. Target positions must
            be distinct.
        Nothing synchronises with the host.
        """
        if isinstance(donor_positions, torch.Tensor):
            donor_positions = donor_positions.cpu().numpy()
        if isinstance(target_positions, torch.Tensor):
            target_positions = target_positions.cpu().numpy()
        sizes = [self._chunk_tokens_of(ch) for ch in chunks]
        pairs, offsets = self._group(donor_positions, target_positions, len(chunks))
        n_all = pairs.shape[1]
        if n_all == 0:
            return
        flags = _lib.scatter_flags(_lib.rows_repeat(np.asarray(donor_positions)))
        cur = torch.cuda.current_stream(self.dev)
        side = self.scatter_stream
        side.wait_stream(cur)  # the caches' earlier users and the pair upload come first
        # Device memory the scatters read on the side stream: marked there, so the caching
        # allocator does not hand it out again before those reads have run.
        for t in (pairs, self._kv_tab, self.block_table, self._inv_freq):
            t.record_stream(side)
        base = pairs.data_ptr()
        # (kv, head, seq) strides of a slot's layer window in elements; then rows, first
        row = self.num_heads * self.head_dim
        strides = _lib.i64_array([0, self.head_dim, row, 0, 0])
        inv = self._inv_freq.data_ptr() if rope else None
        lib = _lib.lib()
        for c, ch in enumerate(chunks):
            lo, hi = int(offsets[c]), int(offsets[c + 1])
            if hi == lo:
                continue
            tc = sizes[c]
            s = self._next
            self._next = (s + 1) % len(self._slots)
            win = self._window(self._slots[s], tc)
            cur.wait_event(self._free[s])  # the last scatter from this slot has run
            win.copy_(ch.view(win.shape), non_blocking=True)
            self._loaded[s].record(cur)
            side.wait_event(self._loaded[s])
            tab = self._slot_tabs[s] if tc == self.chunk_tokens else self._layer_table(
                self._slots[s], tc)
            tab.record_stream(side)
            self._slots[s].record_stream(side)
            strides[0] = self.num_layers * tc * row
            strides[3] = tc
            strides[4] = c * self.chunk_tokens
            rc = lib.sb_composite_scatter_paged_layers(
                self._kv_tab.data_ptr(), self.num_layers, tab.data_ptr(), 1, strides,
                base + 4 * (2 * n_all + lo), base + 4 * lo, base + 4 * (n_all + lo), inv,
                hi - lo, self.num_heads, self.block_size, self.head_dim,
                self.block_table.data_ptr(), self.nb_total, self.block_table.shape[0],
                self._kv_strides, self._dtype_code, flags, side.cuda_stream)
            if rc != _lib.SB_OK:
                raise RuntimeError("sb_composite_scatter_paged_layers failed: "
                                   + lib.sb_last_error_string().decode())
            self._free[s].record(side)
        cur.wait_stream(side)

    def _chunk_tokens_of(self, ch: torch.Tensor) -> int:
        """Tokens in a host chunk after checking its layout; returns T_c."""
        if ch.is_cuda:
            raise ValueError("chunks are host tensors (the loader copies them to the GPU)")
        if not ch.is_pinned():
            raise ValueError("chunks must be in pinned host memory for asynchronous copies")
        if ch.dtype != self.dtype:
            raise TypeError("chunk dtype differs from the caches'")
        if not ch.is_contiguous():
            raise ValueError("chunks must be contiguous [2, L, T, H*D] (KV_2LTD)")
        row = self.num_heads * self.head_dim
        if ch.dim() == 4:
            ok = ch.shape[0] == 2 and ch.shape[1] == self.num_layers and ch.shape[3] == row
        elif ch.dim() == 5:
            ok = (ch.shape[0] == 2 and ch.shape[1] == self.num_layers
                  and ch.shape[3] == self.num_heads and ch.shape[4] == self.head_dim)
        else:
            ok = False
        if not ok:
            raise ValueError(f"chunk must be [2, {self.num_layers}, T, {row}] "
                             f"or [2, {self.num_layers}, T, {self.num_heads}, {self.head_dim}]")
        tc = ch.shape[2]
        if tc <= 0 or tc > self.chunk_tokens:
            raise ValueError(f"chunk holds {tc} tokens; at most {self.chunk_tokens}")
        return tc
