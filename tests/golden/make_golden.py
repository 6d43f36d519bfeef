"""Writes the float64 golden vectors in this directory (numpy only; no torch, no oracle).

The reference repository ships no golden vectors for the KV-reuse path, so these fixtures are
the path's closed forms evaluated independently in float64 on seeded inputs:

  rope_golden.npz       interleaved RoPE of rows at given positions (the formula of the
                        reference's test oracle apply_rope_from_scratch,
                        synapse_kv_connector/tests/test_rope_correction.py:14-31), and the
                        delta correction R(t - d) applied to rows rotated to d
  attention_golden.npz  causal softmax attention of selected rows (dense MHA) and GQA attention
                        over a paged cache, by explicit per-row loops
  scatter_golden.npz    paged and flat scatters by explicit per-pair loops

Inputs are stored as float32 (or int32); expected outputs as float64. Run from the repository
root: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def inv_freq64(base: float, d: int) -> np.ndarray:
    return 1.0 / base ** (np.arange(0, d, 2, dtype=np.float64) / d)


def rope64(x: np.ndarray, pos: np.ndarray, base: float) -> np.ndarray:
    """Rotate x[..., s, :] by pos[s] * inv_freq, interleaved pairs, in float64."""
    d = x.shape[-1]
    f = inv_freq64(base, d)
    theta = pos.astype(np.float64)[:, None] * f[None, :]
    c, s = np.cos(theta), np.sin(theta)
    x = x.astype(np.float64)
    out = np.empty_like(x)
    out[..., 0::2] = x[..., 0::2] * c - x[..., 1::2] * s
    out[..., 1::2] = x[..., 0::2] * s + x[..., 1::2] * c
    return out


def softmax_attn64(q, k, v, pos, scale):
    """Row-by-row causal attention: q [H, D] at position pos attends k/v [H, 0..pos]."""
    scores = np.einsum("hd,hkd->hk", q, k[:, : pos + 1]) * scale
    scores -= scores.max(axis=-1, keepdims=True)
    w = np.exp(scores)
    w /= w.sum(axis=-1, keepdims=True)
    return np.einsum("hk,hkd->hd", w, v[:, : pos + 1])


def make_rope(rng) -> dict:
    out = {}
    for i, (base, d) in enumerate([(10000.0, 64), (1e6, 128), (500.0, 32), (5e5, 128)]):
        heads, n = 2, 8
        raw = rng.standard_normal((heads, n, d)).astype(np.float32)
        dpos = rng.integers(0, 200, n).astype(np.int32)
        tpos = (dpos + rng.integers(-64, 65, n)).astype(np.int32)
        out[f"c{i}_base"] = np.float64(base)
        out[f"c{i}_raw"] = raw
        out[f"c{i}_dpos"] = dpos
        out[f"c{i}_tpos"] = tpos
        # K as cached at the donor positions (rounded to float32 like a stored cache) ...
        out[f"c{i}_k_at_d"] = rope64(raw, dpos, base).astype(np.float32)
        # ... and the exact rows at the target positions
        out[f"c{i}_k_at_t"] = rope64(raw, tpos, base)
        # and the exact correction of the stored rows by (t - d)
        out[f"c{i}_corrected"] = rope64(out[f"c{i}_k_at_d"], tpos - dpos, base)
    return out


def make_attention(rng) -> dict:
    out = {}
    # dense MHA cases: [H, S, D], mask, scale
    for i, (h, s, d) in enumerate([(2, 8, 16), (2, 37, 64), (1, 70, 32)]):
        q = rng.standard_normal((h, s, d)).astype(np.float32)
        k = rng.standard_normal((h, s, d)).astype(np.float32)
        v = rng.standard_normal((h, s, d)).astype(np.float32)
        mask = rng.random(s) < 0.4
        mask[-1] = True
        scale = 1.0 / np.sqrt(d) if i != 2 else 0.3
        exp = np.zeros((h, s, d))
        for p in np.nonzero(mask)[0]:
            exp[:, p] = softmax_attn64(q[:, p].astype(np.float64), k.astype(np.float64),
                                       v.astype(np.float64), int(p), scale)
        out.update({f"d{i}_q": q, f"d{i}_k": k, f"d{i}_v": v, f"d{i}_mask": mask,
                    f"d{i}_scale": np.float64(scale), f"d{i}_out": exp})
    # GQA over a paged cache: kv [NB, 2, Hkv, bs, D], block table, positions, q [R, Hq, D]
    nb, hkv, hq, bs, d, seq = 14, 2, 6, 8, 32, 80
    kv = rng.standard_normal((nb, 2, hkv, bs, d)).astype(np.float32)
    bt = rng.permutation(nb)[: seq // bs].astype(np.int32)
    pos = np.sort(rng.choice(seq, 11, replace=False)).astype(np.int32)
    q = rng.standard_normal((pos.shape[0], hq, d)).astype(np.float32)
    t = np.arange(seq)
    kd = kv[bt[t // bs], 0, :, t % bs, :].transpose(1, 0, 2).astype(np.float64)  # [Hkv, S, D]
    vd = kv[bt[t // bs], 1, :, t % bs, :].transpose(1, 0, 2).astype(np.float64)
    group = hq // hkv
    exp = np.zeros((pos.shape[0], hq, d))
    for r, p in enumerate(pos):
        for h in range(hq):
            exp[r, h] = softmax_attn64(q[r, h][None].astype(np.float64), kd[h // group][None],
                                       vd[h // group][None], int(p), 1.0 / np.sqrt(d))[0]
    out.update({"g_kv": kv, "g_bt": bt, "g_pos": pos, "g_q": q, "g_out": exp})
    return out


def make_scatter(rng) -> dict:
    nb, h, bs, d = 10, 3, 4, 8
    kv = rng.standard_normal((nb, 2, h, bs, d)).astype(np.float32)
    donor = rng.standard_normal((2, h, 20, d)).astype(np.float32)
    bt = np.array([7, 2, 9, 0, 12], dtype=np.int32)  # entry 12 is not a valid block
    dpos = np.array([0, 3, 19, 25, 4, 7, 11, -1, 2], dtype=np.int32)
    tpos = np.array([1, 5, 9, 2, 17, 19, 30, 3, 12], dtype=np.int32)
    exp = kv.astype(np.float64).copy()
    for dp, tp in zip(dpos, tpos):
        if dp < 0 or dp >= donor.shape[2] or tp < 0 or tp // bs >= bt.shape[0]:
            continue
        pb = bt[tp // bs]
        if pb < 0 or pb >= nb:
            continue
        exp[pb, :, :, tp % bs, :] = donor[:, :, dp, :]
    # flat [L, 2, H, S, D]
    tgt = rng.standard_normal((2, 2, h, 16, d)).astype(np.float32)
    dfl = rng.standard_normal((2, 2, h, 12, d)).astype(np.float32)
    fd = np.array([0, 11, 5, 12, 3], dtype=np.int32)
    ft = np.array([15, 0, 7, 2, 16], dtype=np.int32)
    fexp = tgt.astype(np.float64).copy()
    for dp, tp in zip(fd, ft):
        if 0 <= dp < 12 and 0 <= tp < 16:
            fexp[:, :, :, tp, :] = dfl[:, :, :, dp, :]
    return {"p_kv": kv, "p_donor": donor, "p_bt": bt, "p_dpos": dpos, "p_tpos": tpos,
            "p_out": exp, "f_target": tgt, "f_donor": dfl, "f_dpos": fd, "f_tpos": ft,
            "f_out": fexp}


def main() -> None:
    rng = np.random.default_rng(20261201)
    np.savez_compressed(HERE / "rope_golden.npz", **make_rope(rng))
    np.savez_compressed(HERE / "attention_golden.npz", **make_attention(rng))
    np.savez_compressed(HERE / "scatter_golden.npz", **make_scatter(rng))
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()
