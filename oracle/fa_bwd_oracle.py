"""CPU checker for the backward pass: a float64 numpy restatement of the
reference's backward golden.

TEST INFRASTRUCTURE ONLY. tests/ import this module to check the HIP
backward; the product never does.

Follows `golden_bsnd_bwd_from_fwd` / `golden_tnd_bwd_from_fwd` and their helpers
in tests/fa_small_op_golden.py of the reference:
  * P = exp(s - lse) from the forward's LSE (softmax_res_from_fa_lse_bsnd,
    :118-150), s = q.k^T * scale, soft-capped as c * tanh(s / c) (:140-141),
    masked rows/keys set to 0 (:147-149) with the window mask of
    make_window_atten_mask (:34-58);
  * dV = P^T dO, dP = dO V^T, dS = P * (dP - rowsum(dP * P)) * scale
    (tsoftmax_grad :69-72, tbackward_bsnd :181-197), times 1 - tanh^2 with
    soft capping (_softcap_backward_factor :79-86);
  * dQ = dS K, dK = dS^T Q, and dK / dV summed over the g query heads of each
    kv head (sum_gqa_grad :89-100).
Two differences, both on the exact side: q.k^T is formed in float64 here (the
golden rounds it to the input dtype, :137), and ALiBi (which the golden does
not model) enters as the forward defines it: -slope_h * |i + Sk - Sq - j|
added to the soft-capped score.
Inputs are float arrays (the 16-bit values, widened); outputs are float64.
"""
import numpy as np


def _window(sq, sk, causal, wl, wr):
    """normalize_window, tests/fa_small_op_golden.py:21-32."""
    if wl >= sk - 1:
        wl = -1
    if wr >= sq - 1:
        wr = -1
    if causal:
        wr = 0
    return wl, wr


def _visible(sq, sk, causal, wl, wr, chunk=0):
    """Keep-mask (Sq, Sk): bottom-right aligned causal / local window and, with
    attention_chunk c > 0 (v3 API), keys in [c*floor(d/c), c*floor(d/c) + c)."""
    wl, wr = _window(sq, sk, causal, wl, wr)
    i = np.arange(sq)[:, None]
    j = np.arange(sk)[None, :]
    keep = np.ones((sq, sk), dtype=bool)
    d = i + sk - sq
    if wr >= 0:
        keep &= j <= d + wr
    if wl >= 0:
        keep &= j >= d - wl
    if chunk > 0:
        c0 = np.floor_divide(d, chunk) * chunk
        keep &= (j >= c0) & (j < c0 + chunk)
    return keep


def _one(q, k, v, do, lse, *, scale, softcap, causal, window, alibi_row, chunk=0):
    """One sequence. q, do: (H, Sq, D); k, v: (Hk, Sk, D); lse: (H, Sq).
    Returns dq (H, Sq, D), dk, dv (Hk, Sk, D)."""
    H, sq, _ = q.shape
    Hk, sk, _ = k.shape
    g = H // Hk
    kb = np.repeat(k, g, axis=0)  # broadcast_kv_single: head h uses kv head h // g
    vb = np.repeat(v, g, axis=0)
    s = np.matmul(q, kb.transpose(0, 2, 1)) * scale
    t = None
    if softcap > 0.0:
        t = np.tanh(s / softcap)
        s = softcap * t
    if alibi_row is not None:
        i = np.arange(sq)[:, None]
        j = np.arange(sk)[None, :]
        dist = np.abs(i + sk - sq - j).astype(np.float64)
        s = s - alibi_row[:, None, None] * dist[None]
    keep = _visible(sq, sk, causal, *window, chunk=chunk)
    with np.errstate(invalid="ignore", over="ignore"):
        p = np.exp(s - lse[:, :, None])
    p = np.where(keep[None], p, 0.0)
    p = np.where(np.isfinite(lse)[:, :, None], p, 0.0)
    dv = np.matmul(p.transpose(0, 2, 1), do)
    dp = np.matmul(do, vb.transpose(0, 2, 1))
    ds = p * (dp - (dp * p).sum(-1, keepdims=True)) * scale
    if t is not None:
        ds = ds * (1.0 - t * t)
    dq = np.matmul(ds, kb)
    dk = np.matmul(ds.transpose(0, 2, 1), q)
    dk = dk.reshape(Hk, g, sk, -1).sum(1)
    dv = dv.reshape(Hk, g, sk, -1).sum(1)
    return dq, dk, dv


def attention_bwd(q, k, v, dout, lse, *, scale, softcap=0.0, causal=False, window=(-1, -1), alibi=None,
                  cu_seqlens_q=None, cu_seqlens_k=None, chunk=0):
    """Gradients of the forward attention given its LSE.

    Dense: q, dout (B, Sq, H, D); k, v (B, Sk, Hk, D); lse (B, H, Sq).
    Varlen: q, dout (T, H, D); k, v (Tk, Hk, D); lse (H, T) with cu_seqlens_q/k.
    alibi: (H,) or (B, H) slopes or None. Returns float64 dq, dk, dv shaped
    like q, k, v."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    dout = np.asarray(dout, np.float64)
    lse = np.asarray(lse, np.float64)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    if cu_seqlens_q is None:
        B = q.shape[0]
        for b in range(B):
            ar = None if alibi is None else np.asarray(alibi, np.float64).reshape(-1, q.shape[2])[
                b if np.ndim(alibi) == 2 else 0]
            a, bk, c = _one(q[b].transpose(1, 0, 2), k[b].transpose(1, 0, 2), v[b].transpose(1, 0, 2),
                            dout[b].transpose(1, 0, 2), lse[b], scale=scale, softcap=softcap, causal=causal,
                            window=window, alibi_row=ar, chunk=chunk)
            dq[b] = a.transpose(1, 0, 2)
            dk[b] = bk.transpose(1, 0, 2)
            dv[b] = c.transpose(1, 0, 2)
        return dq, dk, dv
    cq = np.asarray(cu_seqlens_q)
    ck = np.asarray(cu_seqlens_k)
    for b in range(len(cq) - 1):
        qs, qe, ks, ke = int(cq[b]), int(cq[b + 1]), int(ck[b]), int(ck[b + 1])
        if qe == qs:
            continue
        ar = None if alibi is None else np.asarray(alibi, np.float64).reshape(-1, q.shape[1])[
            b if np.ndim(alibi) == 2 else 0]
        a, bk, c = _one(q[qs:qe].transpose(1, 0, 2), k[ks:ke].transpose(1, 0, 2), v[ks:ke].transpose(1, 0, 2),
                        dout[qs:qe].transpose(1, 0, 2), lse[:, qs:qe], scale=scale, softcap=softcap,
                        causal=causal, window=window, alibi_row=ar, chunk=chunk)
        dq[qs:qe] = a.transpose(1, 0, 2)
        dk[ks:ke] += bk.transpose(1, 0, 2)
        dv[ks:ke] += c.transpose(1, 0, 2)
    return dq, dk, dv


def softmax_d(out, dout):
    """rowsum(dout * out) in the LSE layout: dense (B, Sq, H, D) -> (B, H, Sq);
    varlen (T, H, D) -> (H, T)."""
    prod = (np.asarray(out, np.float64) * np.asarray(dout, np.float64)).sum(-1)
    if prod.ndim == 3:
        return prod.transpose(0, 2, 1)
    return prod.T
