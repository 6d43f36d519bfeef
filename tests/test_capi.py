"""The C ABI library (no GPU): it loads, exports every function include/semblend_hip.h
declares with the argument counts the ctypes binding uses, and rejects invalid arguments with
SB_ERR_INVALID_ARGUMENT before launching anything."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from semblend_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "semblend_hip.h"


def _declared() -> dict[str, int]:
    """Function name -> parameter count, parsed from the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|int64_t|const char\*)\s+(sb_\w+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_header_declares_the_abi():
    decl = _declared()
    assert "sb_version" in decl and "sb_last_error_string" in decl
    assert set(_lib.SIGNATURES) | set(_lib.SIZE_QUERIES) | {"sb_version", "sb_last_error_string"} \
        == set(decl)


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name, nparams in _declared().items():
        assert hasattr(lib, name), name
        if name in _lib.SIGNATURES:
            assert len(_lib.SIGNATURES[name]) == nparams, name
        if name in _lib.SIZE_QUERIES:
            assert len(_lib.SIZE_QUERIES[name]) == nparams, name


def test_version():
    assert _lib.version().startswith("semblend_hip ") and "gfx950" in _lib.version()


def _i64(*v):
    return (ctypes.c_int64 * len(v))(*v)


def test_invalid_arguments_are_rejected_without_launch():
    lib = _lib.lib()
    fake = 4096  # never dereferenced: validation fails first
    st = _i64(1, 1, 1, 1, 1)
    # bad dtype
    rc = lib.sb_scatter_donor_kv(fake, fake, fake, fake, 4, 1, 1, 8, 4, 4, st, st, 7, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT
    assert b"invalid dtype" in lib.sb_last_error_string()
    # null pointers
    rc = lib.sb_scatter_donor_kv_paged(None, fake, fake, fake, fake, 4, 1, 16, 8, 4, 4, 1, st,
                                       st, 2, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"null" in lib.sb_last_error_string()
    # non-contiguous head_dim
    bad = _i64(1, 1, 1, 1, 2)
    rc = lib.sb_rope_correct_scatter_paged(fake, fake, fake, fake, fake, fake, 4, 1, 16, 8, 4,
                                           4, 1, bad, _i64(1, 1, 1, 1), 2, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"contiguous" in lib.sb_last_error_string()
    # odd head_dim for RoPE
    rc = lib.sb_apply_rope_delta_inplace(fake, fake, fake, None, 3, 5, fake, 1, 16, 7, 4, 1,
                                         _i64(1, 1, 1, 1), 2, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"even" in lib.sb_last_error_string()
    # GQA head counts
    rc = lib.sb_partial_attention_paged(fake, fake, fake, fake, fake, None, 0, 4, 7, 2, 128,
                                        16, 8, 4, 1.0, _i64(1, 1, 1), _i64(1, 1, 1),
                                        _i64(1, 1, 1, 1, 1), 2, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"multiple" in lib.sb_last_error_string()
    # workspace too small for the dense drop-in
    rc = lib.sb_partial_prefill_attention(fake, fake, fake, fake, fake, fake, 8, 2, 64, 128,
                                          0.1, _i64(1, 1, 1), _i64(1, 1, 1), _i64(1, 1, 1),
                                          _i64(1, 1, 1), 2, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"workspace" in lib.sb_last_error_string()
    # more host positions than the launch carries
    many = (ctypes.c_int32 * 257)()
    rc = lib.sb_apply_rope_delta_inplace_host(fake, fake, many, None, 257, 5, fake, 1, 16, 8,
                                              4, 1, _i64(1, 1, 1, 1), 2, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT
    assert b"SB_INLINE_POSITIONS_MAX" in lib.sb_last_error_string()
    # unknown scatter flags (bit 0 is the only one defined)
    rc = lib.sb_scatter_donor_kv_paged_layers(fake, fake, 2, fake, fake, fake, 4, 1, 16, 8, 4,
                                              4, 1, st, _i64(1, 1, 1, 1), 2, 2, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"flags" in lib.sb_last_error_string()
    rc = lib.sb_composite_scatter_paged_layers(fake, 2, fake, 1, _i64(1, 1, 1, 4, 0), fake,
                                               fake, fake, None, 4, 1, 16, 8, fake, 4, 1, st,
                                               2, 4, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"flags" in lib.sb_last_error_string()
    # constant RoPE deltas beyond the kernels' sin/cos range, on both in-place entries
    one = (ctypes.c_int32 * 1)(3)
    for delta in (1 << 31, -(1 << 31), 1 << 40):
        rc = lib.sb_apply_rope_delta_inplace(fake, fake, fake, None, 1, delta, fake, 1, 16, 8,
                                             4, 1, _i64(1, 1, 1, 1), 2, None)
        assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"2^31" in lib.sb_last_error_string()
        rc = lib.sb_apply_rope_delta_inplace_host(fake, fake, one, None, 1, delta, fake, 1, 16,
                                                  8, 4, 1, _i64(1, 1, 1, 1), 2, None)
        assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"2^31" in lib.sb_last_error_string()


def test_device_copy_rejects_bad_sizes_and_alignment():
    lib = _lib.lib()
    rc = lib.sb_device_copy(4096, 8192, 40, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"multiple of 16" in lib.sb_last_error_string()
    rc = lib.sb_device_copy(4097, 8192, 32, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"aligned" in lib.sb_last_error_string()
    rc = lib.sb_device_copy(None, 8192, 32, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"null" in lib.sb_last_error_string()
    assert lib.sb_device_copy(None, None, 0, None) == _lib.SB_OK


def test_grouped_composite_rejects_bad_segments():
    lib = _lib.lib()
    fake = 4096
    st = _i64(1, 1, 1, 4, 0, 1, 1, 1, 4, 0)
    kvs = _i64(1, 1, 1, 1, 1)
    for ends, n in (((100, 300), 300), ((256, 300), 299), ((512, 256), 256)):
        rc = lib.sb_composite_scatter_paged_layers_grouped(
            fake, 2, fake, 2, st, _i64(*ends), fake, fake, None, n, 1, 16, 8, fake, 4, 1, kvs,
            2, 0, None)
        assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"segment" in lib.sb_last_error_string()
    rc = lib.sb_composite_scatter_paged_layers_grouped(
        fake, 2, fake, 17, _i64(*([1] * 85)), _i64(*([0] * 17)), fake, fake, None, 10, 1, 16,
        8, fake, 4, 1, kvs, 2, 0, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"16 donors" in lib.sb_last_error_string()


def test_rope_delta_range_checked_before_dispatch():
    """The Python entry rejects |delta| >= 2^31 before touching any tensor (so a CPU tensor
    gets the range error, not the device error)."""
    import torch

    from semblend_amd import rope_correction as rc

    kv = torch.zeros((2, 2, 1, 4, 8))
    bt = torch.tensor([0, 1], dtype=torch.int32)
    for delta in (1 << 31, -(1 << 31)):
        with pytest.raises(ValueError, match="2\\^31"):
            rc.apply_rope_delta_inplace(kv, bt, [0, 1], delta)
    with pytest.raises(RuntimeError, match="device tensors"):
        rc.apply_rope_delta_inplace(kv, bt, [0, 1], (1 << 31) - 1)


def test_uploads_under_capture(monkeypatch):
    """While the stream is capturing a HIP graph no pinned staging memory can be allocated,
    and a captured host-to-device copy reads its host buffer again at every replay. So
    pinned_upload raises for pageable host data under capture, and keeps an already pinned
    host tensor for the process (the replays read it). Outside capture nothing is kept. The
    pinning and the copy run as CPU stand-ins here (no GPU); the rule is what is checked."""
    import torch

    monkeypatch.setattr(torch.Tensor, "pin_memory", lambda self: self.clone())
    cpu = torch.device("cpu")
    before = len(_lib._CAPTURED_UPLOADS)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    out = _lib.upload_index(torch.arange(5), cpu)
    assert torch.equal(out, torch.arange(5, dtype=torch.int32))
    assert len(_lib._CAPTURED_UPLOADS) == before
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    with pytest.raises(RuntimeError, match="capturing"):
        _lib.upload_index(torch.arange(7), cpu)
    from semblend_amd import rope_correction as rc

    with pytest.raises(RuntimeError, match="capturing"):
        rc._pairs_on_device([(1, 2), (3, 4)], cpu)
    pinned = torch.arange(9, dtype=torch.int32)
    monkeypatch.setattr(torch.Tensor, "is_pinned", lambda self: self is pinned)
    out = _lib.pinned_upload(pinned, cpu)
    assert torch.equal(out, pinned) and _lib._CAPTURED_UPLOADS[-1] is pinned
    assert len(_lib._CAPTURED_UPLOADS) == before + 1
    del _lib._CAPTURED_UPLOADS[before:]


def test_empty_calls_are_no_ops():
    lib = _lib.lib()
    st = _i64(1, 1, 1, 1, 1)
    assert lib.sb_scatter_donor_kv_paged(None, None, None, None, None, 0, 1, 16, 8, 4, 4, 1, st,
                                         st, 2, None) == _lib.SB_OK
    assert lib.sb_apply_rope_delta_inplace(None, None, None, None, 0, 5, None, 1, 16, 8, 4, 1,
                                           _i64(1, 1, 1, 1), 2, None) == _lib.SB_OK
    assert lib.sb_last_error_string() == b""


@pytest.mark.parametrize("dtype,expect_split", [(2, True), (0, False)])
def test_workspace_size_queries(dtype, expect_split):
    # 7B attention workload: 2458 rows, 28/4 heads, 16384 tokens in blocks of 16
    n = _lib.size_query("sb_partial_attention_paged_workspace_size", 2458, 28, 4, 128, 16, 1024,
                        dtype)
    assert (n > 0) == expect_split  # fp32 takes the unsplit VALU kernel
    dense = _lib.size_query("sb_partial_prefill_attention_workspace_size", 4, 1000, 128, dtype)
    assert dense >= 1001 * 4


@pytest.mark.parametrize("heads,seq_len", [(28, 16384), (4, 3000), (32, 8192)])
def test_dense_workspace_covers_every_row_count(heads, seq_len):
    """The dense drop-in splits its key range by the row count its kernels find on the device,
    so its workspace must hold the split-key partials of every count. The requirement of one
    count is the library's own single-call plan for that many rows, read through the paged
    query (block size 32: its chunk cap of 1023 blocks, 32736 keys, does not bind at these
    lengths, so the two plans coincide)."""
    idx = ((seq_len + 1) * 4 + 255) // 256 * 256
    dense = _lib.size_query("sb_partial_prefill_attention_workspace_size", heads, seq_len, 128, 2)
    need = 0
    for rows in list(range(1, seq_len + 1, 128)) + [seq_len]:
        need = max(need, _lib.size_query("sb_partial_attention_paged_workspace_size", rows, heads,
                                         heads, 128, 32, -(-seq_len // 32), 2))
    assert need > 0
    assert dense - idx >= need


def test_kernel_timing_log_without_launches():
    _lib.kernel_timing(True)
    assert _lib.kernel_time("attn_mfma") == (0.0, 0)
    _lib.kernel_timing(False)
    rc = _lib.lib().sb_kernel_timing_read(None, None, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT


def _plan(pos, hq=28, hkv=4, d=128, bs=16, nbps=1024, dtype=2):
    import torch

    p = torch.as_tensor(pos, dtype=torch.int32).contiguous()
    ptr = ctypes.cast(p.data_ptr(), _lib.I32P)
    need = _lib.size_query("sb_partial_attention_paged_plan", ptr, p.numel(), hq, hkv, d, bs,
                           nbps, dtype, None, 0)
    buf = torch.zeros(max(need, 1), dtype=torch.int32)
    got = _lib.size_query("sb_partial_attention_paged_plan", ptr, p.numel(), hq, hkv, d, bs,
                          nbps, dtype, ctypes.cast(buf.data_ptr(), _lib.I32P), need)
    assert got == need
    return buf[:need].tolist()


@pytest.mark.parametrize("seed,rows,sort", [(0, 2458, True), (1, 700, True), (2, 2458, False),
                                            (3, 40, True)])
def test_attention_plan_orders_every_item_longest_first(seed, rows, sort):
    """The host plan of the paged attention (7B shape: 28/4 heads, 16384-token table): its
    split covers the key range in max_chunks chunks that fit the kernel's block-table slice;
    its order is a permutation of every work item of the launch, and the items' key counts
    (recomputed here from the positions, with the kernel's item encoding and chunk rule) never
    increase along it."""
    import torch

    g = torch.Generator("cpu").manual_seed(seed)
    pos = torch.randperm(16384, generator=g)[:rows]
    if sort:
        pos = pos.sort().values
    plan = _plan(pos)
    ks1, ks2, mc = plan[:3]
    order = plan[3:]
    assert ks1 > 0 and ks2 > 0 and ks1 % 64 == 0 and ks2 % 64 == 0 and ks1 <= 1024 * 16
    chunks = 1 if 16384 <= ks1 else 1 + -(-(16384 - ks1) // ks2)
    assert mc == chunks
    group, hkv = 7, 4
    # flattened query rows per workgroup tile, from the workspace the library reports for a
    # one-row call (hkv x 1 tile x mc chunks x tr rows x (head_dim + 2) fp32 values)
    ws1 = _lib.size_query("sb_partial_attention_paged_planned_workspace_size", 1, 28, hkv, 128,
                          max(mc, 2), 2)
    tr = ws1 // (hkv * max(mc, 2) * 130 * 4)
    assert tr in (128, 256) and ws1 == hkv * max(mc, 2) * tr * 130 * 4
    n_tiles = -(-rows * group // tr)
    assert sorted(order) == list(range(mc * n_tiles * hkv))
    kend = [max(int(pos[r // group]) for r in range(t * tr, min((t + 1) * tr, rows * group)))
            + 1 for t in range(n_tiles)]

    def keys(b):
        rest = b // hkv
        tile = n_tiles - 1 - rest % n_tiles
        c = rest // n_tiles
        k0 = 0 if c == 0 else ks1 + (c - 1) * ks2
        k1 = min(k0 + (ks1 if c == 0 else ks2), kend[tile])
        return max(0, -(-(k1 - k0) // 64))

    costs = [keys(b) for b in order]
    assert all(a >= b for a, b in zip(costs, costs[1:]))


def test_attention_plan_edge_cases():
    lib = _lib.lib()
    # fp32 (the VALU kernel): no split, no items
    assert _plan([5, 9, 100], dtype=0) == [0, 0, 0]
    # a capacity below the need, and bad shapes, are refused
    import torch

    p = torch.tensor([1, 2, 3], dtype=torch.int32)
    ptr = ctypes.cast(p.data_ptr(), _lib.I32P)
    small = torch.zeros(4, dtype=torch.int32)
    rc = _lib.size_query("sb_partial_attention_paged_plan", ptr, 3, 28, 4, 128, 16, 64, 2,
                         ctypes.cast(small.data_ptr(), _lib.I32P), 4)
    assert rc == -_lib.SB_ERR_INVALID_ARGUMENT
    assert b"too small" in lib.sb_last_error_string()
    assert _lib.size_query("sb_partial_attention_paged_plan", ptr, 3, 28, 5, 128, 16, 64, 2,
                           None, 0) < 0
    # the planned launch rejects a split that does not match max_chunks, before any launch
    fake = 4096
    rc = lib.sb_partial_attention_paged_planned(
        fake, fake, fake, fake, fake, fake, 12, 8640, 4288, 2, None, 0, 10, 28, 4, 128, 16, 2048,
        1024, 0.1, _i64(1, 1, 1), _i64(1, 1, 1), _i64(1, 1, 1, 1, 1), 2, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"max_chunks" in lib.sb_last_error_string()
    rc = lib.sb_partial_attention_paged_planned(
        fake, fake, fake, fake, fake, fake, 12, 8001, 4288, 3, None, 0, 10, 28, 4, 128, 16, 2048,
        1024, 0.1, _i64(1, 1, 1), _i64(1, 1, 1), _i64(1, 1, 1, 1, 1), 2, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"split" in lib.sb_last_error_string()
    # 10 rows x 7 q-heads per KV head = 1 row tile: 3 chunks x 1 x 4 heads = 12 items
    rc = lib.sb_partial_attention_paged_planned(
        fake, fake, fake, fake, fake, fake, 11, 8640, 4288, 3, None, 0, 10, 28, 4, 128, 16,
        2048, 1024, 0.1, _i64(1, 1, 1), _i64(1, 1, 1), _i64(1, 1, 1, 1, 1), 2, None)
    assert rc == _lib.SB_ERR_INVALID_ARGUMENT and b"num_items" in lib.sb_last_error_string()


def test_projection_workspace_covers_the_split_product():
    """The fused projection's workspace: the RoPE table (rows padded to a multiple of 32, x
    head_dim fp32, rounded up to 256 bytes), plus, when the row count leaves CUs without a
    128 x 128 tile, the fp32 slices of the split hidden dimension (Qwen2.5-7B: 4 slices of
    14 k-steps at 64 and 300 rows, none at 2458)."""
    lib = _lib.lib()
    f = (28 + 2 * 4) * 128
    size = lib.sb_qkv_projection_paged_workspace_size
    assert size(64, 28, 4, 128, 3584, 1) == 64 * 128 * 4 + 4 * 64 * f * 4
    assert size(64, 28, 4, 128, 3584, 0) == 4 * 64 * f * 4
    assert size(300, 28, 4, 128, 3584, 1) == 320 * 128 * 4 + 4 * 300 * f * 4
    assert size(2458, 28, 4, 128, 3584, 1) == 2464 * 128 * 4
    assert size(2458, 28, 4, 128, 3584, 0) == 0
    assert size(0, 28, 4, 128, 3584, 1) == 0
