"""Exact (float64) attention by brute force, written independently of the
C oracle, for pinning it and for writing the golden fixtures.

Every score of a (batch, head) pair is formed at once and the softmax is taken
over the visible keys in one pass, with no key stacks, no online rescale and no
rounding of P. The mask is built the way the reference's small-op golden
builds it, from triangular matrices (tests/fa_small_op_golden.py:21-58 in the
reference): bottom-right aligned causal, sliding window [i + Sk - Sq - wl,
i + Sk - Sq + wr]. GQA maps q head h to kv head h // (H / Hk)
(`broadcast_kv_single`, tests/fa_small_op_golden.py:11-18). ALiBi adds
-slope * |i + Sk - Sq - j| to the scaled (and soft-capped) score. Rows with no
visible key give out = 0, lse = +inf.
"""
import numpy as np


def normalize_window(sq, sk, causal, wl, wr):
    """tests/fa_small_op_golden.py:21-32; returns (wl, wr, is_causal, is_local)."""
    if wl >= sk - 1:
        wl = -1
    if wr >= sq - 1:
        wr = -1
    if causal:
        wr = 0
    is_causal = wl < 0 and wr == 0
    is_local = (wl >= 0 or wr >= 0) and not is_causal
    return wl, wr, is_causal, is_local


def mask_keep(sq, sk, causal=False, window=(-1, -1), chunk=0):
    """(sq, sk) bool, True = key visible (tests/fa_small_op_golden.py:35-58).
    chunk > 0 (v3 attention_chunk) also keeps only keys whose chunk id
    j // chunk equals that of the query's diagonal key i + sk - sq."""
    if chunk > 0:
        d = np.arange(sq)[:, None] + sk - sq
        same = (np.arange(sk)[None, :] // chunk) == (d // chunk)
        return mask_keep(sq, sk, causal, window) & same
    wl, wr, is_causal, is_local = normalize_window(sq, sk, causal, window[0], window[1])
    ones = np.ones((sq, sk))
    off = sk - sq
    if is_causal:
        masked = np.triu(ones, off + 1)
    elif is_local:
        masked = np.zeros((sq, sk))
        if wr >= 0:
            masked = masked + np.triu(ones, wr + 1 + off)
        if wl >= 0:
            masked = masked + np.tril(ones, -wl - 1 + off)
    else:
        masked = np.zeros((sq, sk))
    return masked == 0


def attention(q, k, v, scale, causal=False, window=(-1, -1), alibi=None, softcap=0.0, chunk=0):
    """One sequence. q (Sq, H, D), k (Sk, Hk, D), v (Sk, Hk, Dv), any float;
    alibi (H,) or None. Returns out (Sq, H, Dv) float64, lse (H, Sq) float64."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    sq, h, _ = q.shape
    sk, hk, dv = v.shape
    g = h // hk
    keep = mask_keep(sq, sk, causal, window, chunk)
    out = np.zeros((sq, h, dv))
    lse = np.full((h, sq), np.inf)
    if sk == 0:
        return out, lse
    dist = np.abs(np.arange(sq)[:, None] + sk - sq - np.arange(sk)[None, :])
    for hh in range(h):
        kv = hh // g
        s = (q[:, hh, :] @ k[:, kv, :].T) * scale
        if softcap > 0:
            s = softcap * np.tanh(s / softcap)
        if alibi is not None:
            s = s - float(alibi[hh]) * dist
        s = np.where(keep, s, -np.inf)
        m = s.max(axis=1, keepdims=True)
        rows = np.isfinite(m[:, 0])
        p = np.zeros_like(s)
        p[rows] = np.exp(s[rows] - m[rows])
        l = p.sum(axis=1)
        out[rows, hh, :] = (p[rows] @ v[:, kv, :]) / l[rows, None]
        lse[hh, rows] = np.log(l[rows]) + m[rows, 0]
    return out, lse


def attention_batch(q, k, v, seqlens_k, scale, causal=False, window=(-1, -1), alibi=None, softcap=0.0, chunk=0):
    """q (B, Sq, H, D); k, v (B, >=Sk_b, Hk, D); seqlens_k[b] keys of batch b.
    alibi (H,) or (B, H). Returns out (B, Sq, H, Dv), lse (B, H, Sq)."""
    B = q.shape[0]
    outs, lses = [], []
    for b in range(B):
        al = None
        if alibi is not None:
            al = alibi[b] if np.ndim(alibi) == 2 else alibi
        n = int(seqlens_k[b])
        o, l = attention(q[b], k[b, :n], v[b, :n], scale, causal, window, al, softcap, chunk)
        outs.append(o)
        lses.append(l)
    return np.stack(outs), np.stack(lses)
