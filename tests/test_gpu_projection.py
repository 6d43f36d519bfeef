"""GPU parity: compacted QKV projection (MFMA) against the oracle.

Tolerance (floating point): both sides accumulate in fp32 and round once, in different
summation orders, so an output may differ by one ulp of the output dtype plus the fp32
accumulation difference, bounded here by 2^-16 * sum_k |x_k w_k| of that feature (for
rotated features, of the pair). Away from zero this is the one-ulp bar; near zero it is the
fp32 agreement of two correct GEMMs.
"""

from __future__ import annotations

import pytest
import torch

from oracle import ref_cpu as ref
from semblend_amd import triton_kernels as tk
from tests.helpers import _ulp16, gen, randn

pytestmark = pytest.mark.gpu

ACC_TOL = 2.0 ** -16


def _absdot(x, w):
    return torch.nn.functional.linear(x.float().abs(), w.float().abs())


def _assert_proj_close(got, want, absdot, what=""):
    got, want = got.cpu(), want.cpu()
    assert got.shape == want.shape and got.dtype == want.dtype
    # Non-finite outputs (from non-finite inputs): the oracle's infinity bit for bit, and NaN
    # where it has NaN. NaN bits are not compared with the oracle: torch's CPU rounding writes
    # 0xFFFF from its vectorised path and 0x7FC0 from its scalar one. The library writes 0x7FC0
    # in bf16 from every path (fp16 keeps the NaN's sign).
    nonfinite = ~torch.isfinite(want.float())
    if nonfinite.any():
        w_nan = torch.isnan(want.float())
        w_inf = nonfinite & ~w_nan
        n_diff = int((got[w_inf].view(torch.int16) != want[w_inf].view(torch.int16)).sum())
        g_nan = got[w_nan]
        n_diff += int((~torch.isnan(g_nan.float())).sum())
        if got.dtype == torch.bfloat16:
            n_diff += int((g_nan.view(torch.int16) != 0x7FC0).sum())
        assert n_diff == 0, f"{what}: {n_diff} non-finite outputs differ"
    diff = (got.float() - want.float()).abs()
    mag = torch.maximum(got.float().abs(), want.float().abs())
    allowed = _ulp16(mag, got.dtype) + ACC_TOL * absdot
    bad = (diff > allowed) & ~nonfinite
    bad |= ~torch.isfinite(got.float()) & ~nonfinite
    n_bad = int(bad.sum())
    if n_bad:
        i = bad.nonzero()[0].tolist()
        raise AssertionError(f"{what}: {n_bad} of {bad.numel()} outside the bar; first at {i}: "
                             f"got {float(got[tuple(i)])}, want {float(want[tuple(i)])}, "
                             f"allowed {float(allowed[tuple(i)])}")


def _pair_sum(a):
    """|x||w| sums of each interleaved pair, broadcast to both features of the pair."""
    s = a[..., 0::2] + a[..., 1::2]
    return torch.stack([s, s], dim=-1).reshape(a.shape)


def _case(seq, hidden, hq, hkv, d, n_rows, dtype, seed, nb_extra=5, bs=16, bias=True,
          w_scale=None):
    g = gen(seed)
    x = randn((seq, hidden), dtype, seed + 1)
    f = (hq + 2 * hkv) * d
    w = (randn((f, hidden), torch.float32, seed + 2) *
         (w_scale if w_scale is not None else hidden ** -0.5)).to(dtype)
    b = randn((f,), dtype, seed + 3) if bias else None
    pos = torch.randperm(seq, generator=g)[:n_rows].sort().values.to(torch.int32)
    nbs = (seq + bs - 1) // bs
    bt = torch.randperm(nbs + nb_extra, generator=g)[:nbs].to(torch.int32)
    cache = randn((nbs + nb_extra, 2, hkv, bs, d), dtype, seed + 4)
    return x, w, b, pos, bt, cache


def _check_paged(dev, x, w, b, pos, bt, cache, hq, hkv, d, rope_base, backend="auto"):
    kv_dev = cache.to(dev)
    q = tk.qkv_projection_paged(x.to(dev), w.to(dev), pos.to(dev), kv_dev, bt.to(dev), hq, hkv,
                                d, qkv_bias=None if b is None else b.to(dev),
                                rope_base=rope_base, backend=backend)
    want_kv = cache.clone()
    want_q = ref.qkv_project_paged(x, w, pos, want_kv, bt, hq, hkv, d, qkv_bias=b,
                                   rope_base=rope_base)
    valid = (pos >= 0) & (pos < x.shape[0])
    xs = torch.zeros((pos.shape[0], x.shape[1]), dtype=x.dtype)
    xs[valid] = x[pos[valid].long()]
    ad = _absdot(xs, w)
    qf, kf = hq * d, hkv * d
    ad_q, ad_k, ad_v = ad[:, :qf], ad[:, qf:qf + kf], ad[:, qf + kf:]
    if rope_base is not None:
        ad_q, ad_k = _pair_sum(ad_q), _pair_sum(ad_k)
    _assert_proj_close(q, want_q, ad_q.reshape(q.shape), "Q")
    got_kv = kv_dev.cpu()
    bs = cache.shape[3]
    touched = torch.zeros(cache.shape[0], bs, dtype=torch.bool)
    for r, p in enumerate(pos.tolist()):
        if not (0 <= p < x.shape[0]) or p // bs >= bt.shape[0]:
            continue
        pb, off = int(bt[p // bs]), p % bs
        touched[pb, off] = True
        _assert_proj_close(got_kv[pb, 0, :, off], want_kv[pb, 0, :, off],
                           ad_k[r].reshape(hkv, d), f"K row {r}")
        _assert_proj_close(got_kv[pb, 1, :, off], want_kv[pb, 1, :, off],
                           ad_v[r].reshape(hkv, d), f"V row {r}")
    # every other slot untouched
    keep = ~touched
    assert torch.equal(got_kv.permute(0, 3, 1, 2, 4)[keep].view(torch.int16),
                       cache.permute(0, 3, 1, 2, 4)[keep].view(torch.int16))


BACKENDS = ["fused", "library"]


@pytest.mark.parametrize("backend", BACKENDS)
@pytest.mark.parametrize("rope_base", [None, 1e6], ids=["plain", "rope"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_projection_paged_qwen05b_shape(dev, dtype, rope_base, backend):
    # Qwen2.5-0.5B attention: hidden 896, 14 q heads / 2 KV heads x 64, QKV bias
    x, w, b, pos, bt, cache = _case(300, 896, 14, 2, 64, 77, dtype, 10)
    pos = torch.cat([pos, torch.tensor([-1, 300], dtype=torch.int32)])  # zero Q, no K/V
    _check_paged(dev, x, w, b, pos, bt, cache, 14, 2, 64, rope_base, backend)


@pytest.mark.parametrize("backend", BACKENDS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_projection_paged_nonfinite_rows(dev, dtype, backend):
    """Hidden rows holding a NaN, an infinity, or both infinities: every output of such a row
    is non-finite and must match the oracle's (the same infinity, or NaN: in bf16 the
    library's one NaN 0x7FC0); the other rows keep the usual bar. In the fused kernel the row
    tiles that hold these rows take the exact second packing pass."""
    x, w, b, pos, bt, cache = _case(300, 896, 14, 2, 64, 77, dtype, 50)
    x[pos[3], 5] = float("nan")
    x[pos[10], 7] = float("inf")
    x[pos[20], 0] = float("-inf")
    x[pos[20], 1] = float("inf")
    x[pos[40], 9] = float("-inf")
    _check_paged(dev, x, w, b, pos, bt, cache, 14, 2, 64, 1e6, backend)


@pytest.mark.parametrize("backend", BACKENDS)
def test_projection_paged_qwen7b_full(dev, backend):
    """Qwen2.5-7B attention at the benchmark's size: hidden 3584, 28 / 4 heads x 128, bias,
    2458 computed rows of a 16384-token sequence, RoPE theta 1e6, paged cache of 2048 blocks."""
    import bench

    g = gen(20)
    seq, hidden = 16384, 3584
    pos = bench.recompute_positions(g)
    x, w, b, _, _, _ = _case(64, hidden, 28, 4, 128, 1, torch.bfloat16, 21, nb_extra=0)
    x = randn((seq, hidden), torch.bfloat16, 22)
    bt = torch.randperm(2048, generator=g)[:1024].to(torch.int32)
    cache = randn((2048, 2, 4, 16, 128), torch.bfloat16, 23)
    _check_paged(dev, x, w, b, pos, bt, cache, 28, 4, 128, 1e6, backend)


@pytest.mark.parametrize("backend", BACKENDS)
@pytest.mark.parametrize("n_rows", [64, 300])
def test_projection_paged_qwen7b_few_rows(dev, n_rows, backend):
    """Few rows at the Qwen2.5-7B shape, RoPE theta 1e6: the fused form splits the hidden
    dimension (4 slices of 14 k-steps at 64 and at 300 rows) and its epilogue sums the slices;
    a row without a position gets a zero Q and writes no K/V."""
    x, w, b, pos, bt, cache = _case(4096, 3584, 28, 4, 128, n_rows, torch.bfloat16, 40)
    pos = torch.cat([pos, torch.tensor([-1], dtype=torch.int32)])
    _check_paged(dev, x, w, b, pos, bt, cache, 28, 4, 128, 1e6, backend)


@pytest.mark.parametrize("backend", BACKENDS)
@pytest.mark.parametrize("n_rows", [700, 2100])
def test_projection_paged_llama_shape(dev, n_rows, backend):
    # Llama-3-8B attention: hidden 4096, 32 / 8 heads x 128, no bias, theta 5e5 (700 rows
    # take 256 x 128 tiles, 2100 rows 256 x 256; the 7B test above takes 256 x 192)
    x, w, b, pos, bt, cache = _case(4096, 4096, 32, 8, 128, n_rows, torch.bfloat16, 30,
                                    bias=False)
    _check_paged(dev, x, w, b, pos, bt, cache, 32, 8, 128, 5e5, backend)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_masked_qkv_projection_compacted(dev, dtype):
    """The drop-in masked projection on the MFMA path: computed rows within the bar, reuse
    rows exactly zero; all-true and all-false masks; ragged row count."""
    seq, hidden, h, d = 333, 256, 4, 32
    x = randn((seq, hidden), dtype, 40)
    w = (randn((3 * h * d, hidden), torch.float32, 41) * hidden ** -0.5).to(dtype)
    b = randn((3 * h * d,), dtype, 42)
    for mask in (torch.rand(seq, generator=gen(43)) < 0.3, torch.ones(seq, dtype=torch.bool),
                 torch.zeros(seq, dtype=torch.bool)):
        got = tk.masked_qkv_projection(x.to(dev), w.to(dev), mask.to(dev), b.to(dev)).cpu()
        want = ref.masked_qkv_projection(x, w, mask, b)
        assert torch.all(got[~mask] == 0)
        if mask.any():
            _assert_proj_close(got[mask], want[mask], _absdot(x[mask], w), "masked")


def test_masked_qkv_projection_reference_cases(dev):
    # test_triton_kernels.py:313-385 (hidden 32: torch's GEMM on the device, fp32 as the
    # reference), and fp32 inputs
    x = randn((8, 32), torch.float16, 50)
    w = randn((48, 32), torch.float16, 51)
    b = randn((48,), torch.float16, 52)
    got = tk.masked_qkv_projection(x.to(dev), w.to(dev), torch.ones(8, dtype=torch.bool,
                                                                     device=dev), b.to(dev))
    torch.testing.assert_close(got.cpu(), torch.nn.functional.linear(
        x.float(), w.float(), b.float()).half(), atol=1e-2, rtol=1e-2)
    mask = torch.tensor([True, False] * 4)
    got = tk.masked_qkv_projection(x.to(dev), w.to(dev), mask.to(dev)).cpu()
    assert torch.all(got[~mask] == 0) and not torch.any(torch.all(got[mask] == 0, dim=1))
    xf = randn((20, 64), torch.float32, 53)
    wf = randn((96, 64), torch.float32, 54)
    m = torch.rand(20, generator=gen(55)) < 0.5
    torch.testing.assert_close(tk.masked_qkv_projection(xf.to(dev), wf.to(dev), m.to(dev)).cpu(),
                               ref.masked_qkv_projection(xf, wf, m), atol=1e-5, rtol=1e-5)


def test_projection_paged_rejects(dev):
    x = torch.zeros((16, 96), dtype=torch.bfloat16, device=dev)   # hidden not a multiple of 64
    w = torch.zeros((3 * 2 * 16, 96), dtype=torch.bfloat16, device=dev)
    cache = torch.zeros((4, 2, 2, 16, 16), dtype=torch.bfloat16, device=dev)
    pos = torch.arange(4, dtype=torch.int32, device=dev)
    bt = torch.arange(1, dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        tk.qkv_projection_paged(x, w, pos, cache, bt, 2, 2, 16, backend="fused")
    with pytest.raises(ValueError, match="backend"):
        tk.qkv_projection_paged(x, w, pos, cache, bt, 2, 2, 16, backend="triton")
    with pytest.raises(TypeError):
        tk.qkv_projection_paged(x.float(), w.float(), pos, cache.float(), bt, 2, 2, 16)
    with pytest.raises(ValueError):
        tk.qkv_projection_paged(x, w[:-16], pos, cache, bt, 2, 2, 16)


def test_partial_prefill_layers_paged(dev):
    """Two layers of partial prefill over their own paged caches (Qwen2.5-0.5B attention
    shape, bias, RoPE theta 1e6), each stage against the oracle: the projection to its bar,
    the attention over the oracle-written cache to the attention bar (2e-2), and the output
    projection within 2e-2 * sum_k |Wo[j, k]| + 1 ulp (the attention bar carried through the
    linear map). The second layer runs its attention with the request's host plan."""
    hq, hkv, d, hidden, seq = 14, 2, 64, 896, 400
    x = randn((seq, hidden), torch.bfloat16, 60)
    pos = torch.randperm(seq, generator=gen(61))[:90].sort().values.to(torch.int32)
    nbs = (seq + 15) // 16
    bt = torch.randperm(nbs + 3, generator=gen(62))[:nbs].to(torch.int32)
    for layer in range(2):
        s0 = 70 + 10 * layer
        f = (hq + 2 * hkv) * d
        w = (randn((f, hidden), torch.float32, s0) * hidden ** -0.5).to(torch.bfloat16)
        b = randn((f,), torch.bfloat16, s0 + 1)
        wo = (randn((hidden, hq * d), torch.float32, s0 + 2) * (hq * d) ** -0.5).to(
            torch.bfloat16)
        bo = randn((hidden,), torch.bfloat16, s0 + 3)
        cache = randn((nbs + 3, 2, hkv, 16, d), torch.bfloat16, s0 + 4)  # donor K/V stand-in
        kv_dev = cache.to(dev)
        plan = (tk.plan_partial_attention_paged(pos, hq, hkv, d, 16, bt.shape[0],
                                                torch.bfloat16, dev) if layer == 1 else None)
        res = tk.partial_prefill_layer_paged(
            x.to(dev), w.to(dev), wo.to(dev), pos.to(dev), kv_dev, bt.to(dev), hq, hkv, d,
            qkv_bias=b.to(dev), output_bias=bo.to(dev), rope_base=1e6, plan=plan)
        want_kv = cache.clone()
        want_q = ref.qkv_project_paged(x, w, pos, want_kv, bt, hq, hkv, d, qkv_bias=b,
                                       rope_base=1e6)
        ad = _pair_sum(_absdot(x[pos.long()], w)[:, :hq * d]).reshape(want_q.shape)
        _assert_proj_close(res.query, want_q, ad, f"layer {layer} Q")
        want_attn = ref.partial_attention_paged(want_q, want_kv, bt, pos)
        assert float((res.attention.cpu().float() - want_attn).abs().max()) <= 2e-2
        want_out = torch.nn.functional.linear(want_attn.reshape(len(pos), -1).to(
            torch.bfloat16).float(), wo.float(), bo.float())
        bound = 2e-2 * wo.float().abs().sum(dim=1) + _ulp16(want_out.abs(), torch.bfloat16)
        diff = (res.output.cpu().float() - want_out).abs()
        assert bool((diff <= bound).all()), float((diff - bound).max())


def test_projection_zero_rows(dev):
    x = randn((32, 128), torch.bfloat16, 90).to(dev)
    w = randn(((4 + 2 * 2) * 32, 128), torch.bfloat16, 91).to(dev)
    cache = torch.zeros((4, 2, 2, 16, 32), dtype=torch.bfloat16, device=dev)
    bt = torch.arange(2, dtype=torch.int32, device=dev)
    q = tk.qkv_projection_paged(x, w, torch.zeros(0, dtype=torch.int32, device=dev), cache, bt,
                                4, 2, 32, rope_base=1e4)
    assert q.shape == (0, 4, 32) and torch.all(cache == 0)
