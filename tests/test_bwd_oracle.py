"""Pins the backward checker (oracle/fa_bwd_oracle.py) against torch autograd
in float64: the gradients of a plain attention forward (scores, optional soft
cap and ALiBi, bottom-right causal / local mask, softmax, P.V), differentiated
by autograd, must match the oracle's closed-form backward fed with that
forward's log-sum-exp. Autograd is an independent algorithm, so a dropped
term, a wrong sign, a transposed GQA head map or a missing soft-cap factor
in the oracle fails here."""
import numpy as np
import pytest
import torch

from oracle import fa_bwd_oracle as bo
from tests.golden import brute


def _fwd_autograd(q, k, v, dout, *, scale, softcap, causal, window, alibi, chunk=0):
    """q (H, Sq, D), k/v (Hk, Sk, D) float64 tensors with grad; one sequence."""
    H, sq, _ = q.shape
    Hk, sk, _ = k.shape
    g = H // Hk
    kb = k.repeat_interleave(g, dim=0)
    vb = v.repeat_interleave(g, dim=0)
    s = q @ kb.transpose(1, 2) * scale
    if softcap > 0:
        s = softcap * torch.tanh(s / softcap)
    if alibi is not None:
        i = torch.arange(sq, dtype=torch.float64)[:, None]
        j = torch.arange(sk, dtype=torch.float64)[None, :]
        s = s - alibi[:, None, None] * (i + sk - sq - j).abs()[None]
    # the mask from the brute force's triangular-matrix / chunk-id construction
    keep = torch.from_numpy(brute.mask_keep(sq, sk, causal, window, chunk))
    s = s.masked_fill(~keep[None], float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    out = torch.softmax(s, dim=-1) @ vb
    dq, dk, dv = torch.autograd.grad(out, (q, k, v), dout)
    return lse.detach(), out.detach(), dq, dk, dv


CASES = [
    # H, Hk, Sq, Sk, D, causal, window, softcap, alibi
    (4, 4, 33, 33, 16, True, (-1, -1), 0.0, False),
    (8, 2, 17, 40, 32, True, (-1, -1), 0.0, False),       # GQA, Sk > Sq (bottom-right)
    (4, 1, 30, 30, 16, False, (7, 3), 0.0, False),        # local window
    (4, 2, 25, 25, 8, True, (5, 0), 30.0, False),         # SWA + soft cap
    (6, 3, 20, 28, 16, False, (-1, -1), 2.0, False),      # strong soft cap
    (4, 4, 19, 19, 16, True, (-1, -1), 0.0, True),        # ALiBi
    (8, 4, 12, 50, 24, False, (10, 10), 5.0, True),       # everything
    (4, 2, 40, 40, 16, True, (-1, -1), 0.0, False, 8),    # attention_chunk
    (4, 4, 23, 37, 16, False, (-1, -1), 0.0, False, 10),  # chunk, non-causal, Sk > Sq
    (4, 2, 18, 30, 8, True, (6, 0), 3.0, True, 5),        # chunk with window, soft cap, ALiBi
]


@pytest.mark.parametrize("case", CASES, ids=[str(i) for i in range(len(CASES))])
def test_oracle_bwd_matches_autograd(case):
    H, Hk, sq, sk, D, causal, window, softcap, use_alibi = case[:9]
    chunk = case[9] if len(case) > 9 else 0
    g = torch.Generator().manual_seed(sum(case[:5]))
    q = torch.randn(H, sq, D, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.randn(Hk, sk, D, generator=g, dtype=torch.float64, requires_grad=True)
    v = torch.randn(Hk, sk, D, generator=g, dtype=torch.float64, requires_grad=True)
    dout = torch.randn(H, sq, D, generator=g, dtype=torch.float64)
    alibi = torch.rand(H, generator=g, dtype=torch.float64) * 0.5 if use_alibi else None
    scale = D ** -0.5
    lse, out, dq, dk, dv = _fwd_autograd(q, k, v, dout, scale=scale, softcap=softcap, causal=causal, window=window,
                                         alibi=alibi, chunk=chunk)
    # dense layout: (B=1, S, H, D)
    to_bshd = lambda t: t.detach().numpy().transpose(1, 0, 2)[None]
    rq, rk, rv = bo.attention_bwd(to_bshd(q), to_bshd(k), to_bshd(v), to_bshd(dout), lse.numpy()[None],
                                  scale=scale, softcap=softcap, causal=causal, window=window,
                                  alibi=None if alibi is None else alibi.numpy(), chunk=chunk)
    for got, ref in ((rq, dq), (rk, dk), (rv, dv)):
        np.testing.assert_allclose(got[0].transpose(1, 0, 2), ref.numpy(), rtol=1e-9, atol=1e-10)
    # the dsum helper is rowsum(dout * out)
    sd = bo.softmax_d(to_bshd(out), to_bshd(dout))
    np.testing.assert_allclose(sd[0], (out * dout).sum(-1).numpy(), rtol=1e-12, atol=1e-12)


def test_oracle_bwd_varlen_equals_per_sequence_dense():
    """Varlen slices (including an empty sequence) give the dense result of each slice."""
    rng = np.random.default_rng(5)
    H, Hk, D = 4, 2, 16
    lq, lk = [5, 0, 9, 3], [7, 4, 9, 12]
    cq = np.concatenate([[0], np.cumsum(lq)])
    ck = np.concatenate([[0], np.cumsum(lk)])
    q = rng.standard_normal((cq[-1], H, D))
    k = rng.standard_normal((ck[-1], Hk, D))
    v = rng.standard_normal((ck[-1], Hk, D))
    do = rng.standard_normal((cq[-1], H, D))
    lse = rng.standard_normal((H, cq[-1])) + 3.0
    dq, dk, dv = bo.attention_bwd(q, k, v, do, lse, scale=0.25, causal=True, cu_seqlens_q=cq, cu_seqlens_k=ck)
    for b in range(4):
        qs, qe, ks, ke = cq[b], cq[b + 1], ck[b], ck[b + 1]
        if qe == qs:
            assert not dk[ks:ke].any() and not dv[ks:ke].any()
            continue
        a, bk, c = bo.attention_bwd(q[None, qs:qe], k[None, ks:ke], v[None, ks:ke], do[None, qs:qe],
                                    lse[None, :, qs:qe], scale=0.25, causal=True)
        np.testing.assert_array_equal(dq[qs:qe], a[0])
        np.testing.assert_array_equal(dk[ks:ke], bk[0])
        np.testing.assert_array_equal(dv[ks:ke], c[0])


def test_oracle_bwd_empty_rows_have_zero_grad():
    """Rows with no visible key (lse = +inf, out = 0) contribute nothing."""
    rng = np.random.default_rng(6)
    q = rng.standard_normal((1, 6, 2, 8))
    k = rng.standard_normal((1, 3, 2, 8))
    v = rng.standard_normal((1, 3, 2, 8))
    do = rng.standard_normal((1, 6, 2, 8))
    # causal with Sq=6 > Sk=3: rows 0..2 see no key (bottom-right alignment)
    lse = np.full((1, 2, 6), np.inf)
    lse[:, :, 3:] = 1.0
    dq, dk, dv = bo.attention_bwd(q, k, v, do, lse, scale=0.3, causal=True)
    assert not dq[0, :3].any()
    assert dq[0, 3:].any()
