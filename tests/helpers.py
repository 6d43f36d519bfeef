"""Comparison helpers and seeded input builders shared by the tests."""

from __future__ import annotations

import torch

# Tolerances of the parity bar.
# RoPE rotates interleaved pairs (e, o); every output element is e*c -/+ o*s, so its rounding
# error is set by the pair's norm |(e, o)|, not by the element itself. Where the exact result
# cancels to far below that norm, the reference's own fp32 arithmetic (products rounded to
# fp32, cos/sin within 1 ulp) only fixes it to ~2^-23 of the norm, and a last-bit difference
# in cos or sin between two libraries moves it by that much. The bars are therefore:
ROPE_F32_RTOL = 1e-5   # fp32: |got - want| <= 1e-5 * max(|want|, 0.1 * pair_norm)
ROPE_16_ULPS = 1       # bf16/fp16: within one ulp, or
ROPE_16_NORM_TOL = 2.0 ** -21  # |got - want| <= 2^-21 * pair_norm (fp32-level agreement)
ATTN_16_ATOL = 2e-2    # attention, bf16/fp16 outputs vs an fp32 reference: 2e-2 absolute
# ... and, per output row, relative to that row's scale: at long contexts the outputs shrink
# like 1/sqrt(keys), so an absolute 2e-2 alone would accept a row that lost part of its key
# range. The kernel's own error (Q and P rounded to the input type, output rounded once) is
# about 2^-8 of the row's largest element; 2^-6 leaves a factor of four.
ATTN_16_ROW_RTOL = 2.0 ** -6
ATTN_F32_ATOL = 1e-4   # attention, fp32 (the reference suite's own tolerance)
ATTN_F32_RTOL = 1e-3


def gen(seed: int) -> torch.Generator:
    return torch.Generator("cpu").manual_seed(seed)


def randn(shape, dtype, seed: int) -> torch.Tensor:
    """N(0,1) drawn in fp32 on the host from ``seed`` and rounded to ``dtype``."""
    return torch.randn(shape, generator=gen(seed), dtype=torch.float32).to(dtype)


def _ordered16(x: torch.Tensor) -> torch.Tensor:
    """Map 16-bit float bit patterns to integers whose difference counts ulps."""
    bits = x.contiguous().view(torch.int16).to(torch.int32)
    mag = bits & 0x7FFF
    return torch.where(bits < 0, -mag, mag)


def ulp_distance(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    assert a.dtype == b.dtype and a.dtype in (torch.bfloat16, torch.float16)
    return (_ordered16(a) - _ordered16(b)).abs()


def pair_norm(x: torch.Tensor) -> torch.Tensor:
    """Norm of each interleaved pair (x[2i], x[2i+1]), broadcast to both elements."""
    xf = x.float()
    n = torch.sqrt(xf[..., 0::2] ** 2 + xf[..., 1::2] ** 2)
    return torch.stack([n, n], dim=-1).reshape(xf.shape)


def _ulp16(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Spacing of dtype (bf16 or fp16) at magnitude |x| (normal range)."""
    mant = 7 if dtype == torch.bfloat16 else 10
    e = torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -14)))
    return torch.pow(2.0, e - mant)


def assert_rope_close(got: torch.Tensor, ref: torch.Tensor, composed: bool = False) -> dict:
    """RoPE parity bar (see the constants above). ``composed``: rows rotated several times
    with a rounding to the dtype in between; a rounding that falls differently in an
    intermediate step then carries through, so the bound is one ulp of the pair norm.
    Returns element counts per clause, plus ``total``: for 16-bit dtypes ``exact``,
    ``within_1ulp`` (1 ulp apart, not equal) and ``norm_only`` (more than 1 ulp apart, within
    2^-21 of the pair norm); for fp32 ``exact``, ``within_rel`` (not equal, within 1e-5 of
    |want|) and ``floor_only`` (outside 1e-5 |want|, within the 1e-5 * 0.1 |pair| floor)."""
    got = got.cpu()
    ref = ref.cpu()
    assert got.shape == ref.shape and got.dtype == ref.dtype
    diff = (got.float() - ref.float()).abs()
    norm = pair_norm(ref)
    if got.dtype == torch.float32:
        allowed = ROPE_F32_RTOL * torch.maximum(ref.abs(), 0.1 * norm)
        bad = diff > allowed
        by_rel = diff <= ROPE_F32_RTOL * ref.abs()
        stats = {"total": bad.numel(), "exact": int((diff == 0).sum()),
                 "within_rel": int(((diff > 0) & by_rel).sum()),
                 "floor_only": int((~by_rel & ~bad).sum())}
    else:
        ulps = ulp_distance(got, ref)
        by_norm = diff <= ROPE_16_NORM_TOL * norm
        ok = (ulps <= ROPE_16_ULPS) | by_norm
        if composed:
            ok |= diff <= _ulp16(norm, got.dtype)
        bad = ~ok
        stats = {"total": bad.numel(), "exact": int((ulps == 0).sum()),
                 "within_1ulp": int(((ulps > 0) & (ulps <= ROPE_16_ULPS)).sum()),
                 "norm_only": int(((ulps > ROPE_16_ULPS) & by_norm).sum())}
    n_bad = int(bad.sum())
    if n_bad:
        i = bad.nonzero()[0].tolist()
        raise AssertionError(
            f"{n_bad} of {bad.numel()} elements outside the RoPE bar; first at {i}: "
            f"got {float(got[tuple(i)])}, want {float(ref[tuple(i)])}, "
            f"pair norm {float(norm[tuple(i)])}")
    return stats


def assert_bit_exact(got: torch.Tensor, ref: torch.Tensor) -> None:
    got = got.cpu()
    ref = ref.cpu()
    assert got.shape == ref.shape and got.dtype == ref.dtype
    if got.dtype in (torch.bfloat16, torch.float16):
        eq = torch.equal(got.view(torch.int16), ref.view(torch.int16))
    elif got.dtype == torch.float32:
        eq = torch.equal(got.view(torch.int32), ref.view(torch.int32))
    else:
        eq = torch.equal(got, ref)
    if not eq:
        diff = (got.float() != ref.float()).nonzero()
        raise AssertionError(f"not bit-exact: {diff.shape[0]} elements differ, first {diff[:4]}")


def attn_row_violations(got: torch.Tensor, ref_f32: torch.Tensor) -> torch.Tensor:
    """Boolean per output row (all dims but the last): whether the row misses the per-row
    relative bar max|got - want| <= ATTN_16_ROW_RTOL * max|want_row| (a row whose reference
    is all zeros must be exactly zero)."""
    g = got.float().reshape(-1, got.shape[-1])
    w = ref_f32.float().reshape(-1, ref_f32.shape[-1])
    scale = w.abs().amax(dim=1)
    err = (g - w).abs().amax(dim=1)
    return err > ATTN_16_ROW_RTOL * scale + 1e-30


def assert_attn_close(got: torch.Tensor, ref_f32: torch.Tensor) -> None:
    """Attention parity: fp32 outputs at the reference suite's bar; bf16/fp16 outputs within
    2e-2 absolute of the fp32 reference and within the per-row relative
    bar ATTN_16_ROW_RTOL."""
    got = got.cpu()
    if got.dtype == torch.float32:
        torch.testing.assert_close(got, ref_f32, atol=ATTN_F32_ATOL, rtol=ATTN_F32_RTOL)
    else:
        err = (got.float() - ref_f32).abs().max().item() if got.numel() else 0.0
        assert err <= ATTN_16_ATOL, f"max abs error {err} > {ATTN_16_ATOL}"
        if got.numel():
            bad = attn_row_violations(got, ref_f32)
            if bool(bad.any()):
                g = got.float().reshape(-1, got.shape[-1])
                w = ref_f32.float().reshape(-1, got.shape[-1])
                i = int(bad.nonzero()[0])
                ratio = float((g[i] - w[i]).abs().max() / w[i].abs().max().clamp_min(1e-30))
                raise AssertionError(
                    f"{int(bad.sum())} of {bad.numel()} rows outside the per-row bar; first row "
                    f"{i}: max err / max|want| = {ratio:.4g} > {ATTN_16_ROW_RTOL:.4g}")


def recompute_set(seq_len: int, n_total: int, seed: int, chunk: int = 256,
                  n_chunks: int = 2) -> torch.Tensor:
    """Recompute positions: the first ``chunk`` tokens, ``n_chunks`` random whole chunks (not
    the first), and the rest drawn uniformly without replacement from what remains. Sorted,
    int32. With seq_len=16384, n_total=2458 this is the 15% set of the 7B attention workload.
    """
    g = gen(seed)
    num_chunks = seq_len // chunk
    chosen = torch.randperm(num_chunks - 1, generator=g)[:n_chunks] + 1
    mask = torch.zeros(seq_len, dtype=torch.bool)
    mask[:chunk] = True
    for c in chosen.tolist():
        mask[c * chunk:(c + 1) * chunk] = True
    rest = (~mask).nonzero().flatten()
    n_rest = max(0, n_total - int(mask.sum()))
    pick = rest[torch.randperm(rest.numel(), generator=g)[:n_rest]]
    mask[pick] = True
    return mask.nonzero().flatten().to(torch.int32)
