"""GPU parity of whole pipelines against the oracle:

* the one-layer Qwen2.5-0.5B pipeline (fp32, 1024 tokens): scatter into a permuted paged
  cache, per-token RoPE deltas in [-64, 64] applied in place, 154-row GQA attention over that
  same cache; every step checked, and the RoPE step also through ``rope_correct_k`` on the
  flat donor K and the dense drop-in attention on GQA-expanded K/V;
* the single-layer orchestrator ``partial_prefill`` on the reference suite's own cases
  (synapse_kv_connector/tests/test_triton_kernels.py:504-762: basic, full reuse, no reuse,
  sparse reuse, timing fields) in fp16 as there, and in bf16 and fp32, plus a larger bf16
  case that takes the MFMA projection;
* the full-size Llama-3-8B batch (32 layers, four requests of 8K-32K tokens, deltas in
  [-4096, 4096]): V bit-exact and K within the RoPE bar on sampled pairs of every layer,
  attention on sampled rows of every request in two layers.
"""

from __future__ import annotations

import pytest
import torch

import bench
from oracle import ref_cpu as ref
from semblend_amd import rope_correction as rc
from semblend_amd import triton_kernels as tk
from tests.helpers import (ATTN_F32_ATOL, ATTN_F32_RTOL, ATTN_16_ATOL, assert_attn_close,
                           assert_bit_exact, assert_rope_close, gen, randn)

pytestmark = pytest.mark.gpu


# ---- Qwen2.5-0.5B one-layer pipeline ------------------------------------------------------

def test_qwen05b_pipeline_step_by_step(dev):
    inp = bench.qwen05b_pipeline_inputs(seed=0)
    c = bench.QWEN05B
    assert inp["deltas"].abs().max() <= 64 and inp["rows"].unique().numel() == 154
    # (1) scatter, bit-exact
    want = inp["cache"].clone()
    ref.scatter_donor_kv_paged(want, inp["donor"], inp["block_table"], inp["positions"],
                               inp["positions"])
    kv = inp["cache"].to(dev)
    bt = inp["block_table"].to(dev)
    pos = inp["positions"].to(dev)
    tk.scatter_donor_kv_paged(kv, inp["donor"].to(dev), bt, pos, pos)
    assert_bit_exact(kv, want)
    # (2) per-token RoPE, one in-place call per distinct delta; V untouched
    groups = bench.delta_groups(inp["deltas"])
    assert 100 < len(groups) <= 128
    for dl, where in groups:
        n_want = ref.apply_rope_delta_inplace(want, inp["block_table"], where, dl,
                                              rope_base=c["theta"])
        n_got = rc.apply_rope_delta_inplace(kv, bt, where, dl, rope_base=c["theta"])
        assert n_got == n_want == len(where)
    got = kv.cpu()
    assert_bit_exact(got[:, 1], want[:, 1])
    assert_rope_close(got[:, 0], want[:, 0])
    # the same rotation applied to the flat donor K (rope_correct_k) lands the same rows
    d = inp["positions"]
    t = d + inp["deltas"].to(torch.int32)
    k_flat = rc.rope_correct_k(inp["donor"][0].to(dev), d.to(dev), t.to(dev), head_dim=64,
                               rope_base=c["theta"])
    k_want = ref.rope_correct_k(inp["donor"][0], d, t, head_dim=64, rope_base=c["theta"])
    assert_rope_close(k_flat, k_want)
    k_paged, _ = ref.gather_paged_kv(got, inp["block_table"], c["ctx"])
    assert_bit_exact(k_paged, k_flat.cpu())
    # (3) 154-row GQA attention over the corrected cache
    out = tk.partial_prefill_attention_paged(inp["q"].to(dev), kv, bt, inp["rows"].to(dev))
    want_attn = ref.partial_attention_paged(inp["q"], want, inp["block_table"], inp["rows"])
    assert_attn_close(out, want_attn)
    # the dense drop-in on the GQA-expanded cache gives the same rows, zeros elsewhere
    g = c["hq"] // c["hkv"]
    kd, vd = ref.gather_paged_kv(got, inp["block_table"], c["ctx"])
    qd = torch.zeros((c["hq"], c["ctx"], c["d"]))
    qd[:, inp["rows"].long()] = inp["q"].permute(1, 0, 2)
    mask = torch.zeros(c["ctx"], dtype=torch.bool)
    mask[inp["rows"].long()] = True
    dense = tk.partial_prefill_attention(qd.to(dev), kd.repeat_interleave(g, 0).to(dev),
                                         vd.repeat_interleave(g, 0).to(dev), mask.to(dev))
    dense = dense.cpu()
    assert_attn_close(dense[:, inp["rows"].long()].permute(1, 0, 2), want_attn)
    assert not bool(dense[:, ~mask].any())


def test_qwen05b_pipeline_function_matches_oracle(dev):
    """The bench's pipeline function run through the HIP entry points and through the oracle
    (the CPU baseline it times) on another seed."""
    inp = bench.qwen05b_pipeline_inputs(seed=3)
    kv, out = bench.qwen05b_pipeline(tk, rc, inp, device=dev)
    kv_want, out_want = bench.qwen05b_pipeline(ref, ref, inp)
    got = kv.cpu()
    assert_bit_exact(got[:, 1], kv_want[:, 1])
    assert_rope_close(got[:, 0], kv_want[:, 0])
    assert_attn_close(out, out_want)


# ---- partial_prefill, the single-layer orchestrator ---------------------------------------

def _prefill_case(name: str, dtype: torch.dtype, seed: int):
    """The reference suite's cases (same sizes, masks and pairs; seeded N(0,1) inputs in the
    reference's unscaled form), and a larger one at a realistic scale."""
    g = gen(seed)

    def rn(*shape, scale=1.0):
        return (torch.randn(shape, generator=g) * scale).to(dtype)

    if name == "basic":
        s, hid, h, d, layers, dl = 8, 32, 4, 8, 2, 8
        dp = torch.tensor([0, 1, 2, 3]); tp = dp.clone()
        cm = torch.tensor([False] * 4 + [True] * 4)
    elif name == "full_reuse":
        s, hid, h, d, layers, dl = 4, 16, 2, 8, 1, 4
        dp = torch.arange(s); tp = dp.clone()
        cm = torch.zeros(s, dtype=torch.bool)
    elif name == "no_reuse":
        s, hid, h, d, layers, dl = 4, 16, 2, 8, 1, 4
        dp = torch.zeros(0, dtype=torch.int64); tp = dp.clone()
        cm = torch.ones(s, dtype=torch.bool)
    elif name == "sparse":
        s, hid, h, d, layers, dl = 16, 32, 4, 8, 2, 10
        dp = torch.tensor([0, 2, 4, 6, 8]); tp = torch.tensor([0, 3, 6, 9, 12])
        cm = torch.ones(s, dtype=torch.bool)
        cm[tp] = False
    elif name == "timing":
        s, hid, h, d, layers, dl = 64, 128, 8, 16, 4, 32
        dp = torch.arange(16); tp = dp.clone()
        cm = torch.ones(s, dtype=torch.bool)
        cm[:16] = False
    elif name == "large":
        s, hid, h, d, layers, dl = 384, 512, 8, 64, 2, 384
        perm = torch.randperm(s, generator=g)
        cm = torch.ones(s, dtype=torch.bool)
        cm[perm[:270]] = False
        tp = (~cm).nonzero().flatten()
        dp = torch.randperm(dl, generator=g)[:tp.numel()]
        hs = rn(s, hid)
        donor = rn(layers, 2, h, dl, d)
        wq = rn(3 * h * d, hid, scale=hid ** -0.5)
        wo = rn(hid, h * d, scale=(h * d) ** -0.5)
        return hs, donor, wq, wo, dp.to(torch.int32), tp.to(torch.int32), cm, h, d
    else:
        raise ValueError(name)
    hs = rn(s, hid)
    donor = rn(layers, 2, h, dl, d)
    wq = rn(3 * h * d, hid)
    wo = rn(hid, h * d)
    return hs, donor, wq, wo, dp.to(torch.int32), tp.to(torch.int32), cm, h, d


def _ulp(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    if dtype == torch.float32:
        return x.abs() * 2.0 ** -23 + 1e-38
    mant = 7 if dtype == torch.bfloat16 else 10
    e = torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -14)))
    return torch.pow(2.0, e - mant)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", ["basic", "full_reuse", "no_reuse", "sparse", "timing",
                                  "large"])
def test_partial_prefill_matches_oracle(dev, case, dtype):
    seed = {"basic": 1, "full_reuse": 2, "no_reuse": 3, "sparse": 4, "timing": 5, "large": 6}
    hs, donor, wq, wo, dp, tp, cm, h, d = _prefill_case(case, dtype, seed=seed[case])
    res = tk.partial_prefill(hs.to(dev), donor.to(dev), wq.to(dev), wo.to(dev), dp.to(dev),
                             tp.to(dev), cm.to(dev), h, d)
    out_w, kv_w, computed, reused, ratio = ref.partial_prefill(hs, donor, wq, wo, dp, tp, cm,
                                                               h, d)
    # the reference suite's structural assertions
    assert isinstance(res, tk.PartialPrefillResult)
    assert (res.positions_computed, res.positions_reused) == (computed, reused)
    assert res.computation_ratio == pytest.approx(ratio, abs=1e-6)
    assert res.output.shape == out_w.shape and res.output.dtype == dtype
    assert res.kv_cache.shape == kv_w.shape and res.kv_cache.dtype == dtype
    assert res.total_time_ms > 0 and res.scatter_time_ms >= 0
    assert res.projection_time_ms >= 0 and res.attention_time_ms >= 0
    out = res.output.cpu()
    kv = res.kv_cache.cpu()
    # donor rows copied bit-exact into every layer (reference: exact equality)
    reuse = (~cm).nonzero().flatten()
    for i in range(dp.numel()):
        assert_bit_exact(kv[:, :, :, int(tp[i])], donor[:, :, :, int(dp[i])])
    # positions neither reused nor computed stay zero; reuse rows of the output are zero
    untouched = torch.ones(cm.numel(), dtype=torch.bool)
    untouched[cm] = False
    untouched[tp.long()] = False
    assert not bool(kv[:, :, :, untouched].any())
    assert not bool(out[reuse].any())
    # new K/V of the computed rows (same in every layer): fp32 projection rounded once; two
    # correct GEMMs may round a near-tie apart by one ulp of the dtype
    comp = cm.nonzero().flatten()
    if comp.numel():
        got_kv = kv[:, :, :, comp].float()
        want_kv = kv_w[:, :, :, comp].float()
        dot = torch.nn.functional.linear(hs.float().abs(), wq.float().abs())  # sum |x w|
        kvbound = dot[comp][:, h * d:].reshape(-1, 2, h, d).permute(1, 2, 0, 3)
        tol = _ulp(want_kv, dtype) + 2.0 ** -16 * kvbound.unsqueeze(0)
        assert bool(((got_kv - want_kv).abs() <= tol).all()), "new K/V outside the bar"
        # output rows: the attention bar carried through the output projection, plus an
        # ulp of the output for the final rounding
        # (attention rows are convex combinations of V rows, so |attn| <= max |V|)
        attn_bar = ATTN_16_ATOL if dtype != torch.float32 else ATTN_F32_ATOL
        rel = 0.0 if dtype != torch.float32 else ATTN_F32_RTOL
        vmax = float(kv_w[0, 1].float().abs().max())
        bound = (attn_bar + rel * vmax) * wo.float().abs().sum(dim=1)
        diff = (out[comp].float() - out_w[comp].float()).abs()
        tol = bound.unsqueeze(0) + _ulp(out_w[comp].float(), dtype)
        assert bool((diff <= tol).all()), \
            f"output outside the bar: max excess {float((diff - tol).max())}"


# ---- Llama-3-8B batch at full size --------------------------------------------------------

def test_llama3_8b_batch_full_size(dev):
    """The benched batch exactly: 32 layers, requests of 8192/16384/24576/32768 tokens with
    10/15/20/30% recompute and chunk-constant deltas in [-4096, 4096], pool of 8192 blocks.
    After one RoPE scatter step: for 192 sampled pairs per request, the cache rows of every
    layer against the oracle (V bit-exact, K within the RoPE bar); then batched attention of
    layers 0 and 31, 48 sampled rows per request against the oracle."""
    from semblend_amd.batch import KVReuseBatch

    caches, reqs, theta = bench.llama_batch(dev)
    c = bench.LLAMA
    assert [int(r.block_table.numel()) * 16 for r in reqs] == list(c["ctx"])
    batch = KVReuseBatch(caches, reqs, rope_base=theta)
    batch.scatter_rope()
    torch.cuda.synchronize()
    g = gen(77)
    for r in reqs:
        n = r.donor_positions.numel()
        sel = torch.randperm(n, generator=g)[:192].to(dev)
        d = r.donor_positions[sel].long()
        t = r.target_positions[sel].long()
        assert int((t - d).abs().max()) <= 4096
        pb = r.block_table[t // 16].long()
        off = t % 16
        d_cpu, t_cpu = d.cpu().to(torch.int32), t.cpu().to(torch.int32)
        idx = torch.arange(d.numel(), dtype=torch.int32)
        for layer in range(c["layers"]):
            got = caches[layer][pb, :, :, off, :].cpu()          # [n, 2, H, D]
            donor_rows = r.donor_kvs[layer][:, :, d, :].cpu()     # [2, H, n, D]
            assert_bit_exact(got[:, 1], donor_rows[1].permute(1, 0, 2))
            # oracle: row i rotated by t_i - d_i (rope_correct_k on the gathered rows)
            k_want = ref.rope_correct_k(donor_rows[0], idx, idx + (t_cpu - d_cpu),
                                        head_dim=c["d"], rope_base=theta)
            assert_rope_close(got[:, 0], k_want.permute(1, 0, 2))
    q = randn((batch.num_rows, c["hq"], c["d"]), torch.bfloat16, 78).to(dev)
    for layer in (0, c["layers"] - 1):
        out = batch.attention(layer, q).cpu()
        kv = caches[layer].cpu()
        for i, r in enumerate(reqs):
            a = batch.row_offsets[i]
            nr = r.compute_positions.numel()
            rows = torch.randperm(nr, generator=g)[:48].sort().values
            pos = r.compute_positions.cpu()[rows]
            want = ref.partial_attention_paged(q[a:a + nr].cpu()[rows], kv,
                                               r.block_table.cpu(), pos)
            assert_attn_close(out[a + rows], want)
        del kv
