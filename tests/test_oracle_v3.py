"""Pins the oracle's v3 kvcache extensions (attention_chunk, rotary_seqlens,
cache_leftpad, ragged q and ragged new tokens) before they are trusted as
the checker. CPU only.

The reference kernels reject these arguments, so the semantics are the v3
docstring's (README.md:311-401 of the reference). Each test checks the
oracle against something it does not share code with: the float64 brute force
(tests/golden/brute.py builds the chunk mask from chunk ids, the C oracle
from interval bounds), closed forms, the already pinned dense kvcache path, or
an invariance that an off-by-one in an offset would break.
"""
import numpy as np
import pytest

from oracle import fa_oracle as orc
from tests.golden import brute
from tests.test_oracle import NT, check_vs_brute, f, rbits, rope_tables


@pytest.mark.parametrize("case", [
    # Sq, Sk, causal, window, chunk
    (16, 16, True, (-1, -1), 4),
    (7, 300, True, (-1, -1), 64),      # chunk boundaries inside a key stack
    (5, 1030, False, (-1, -1), 512),   # chunk = key stack, non-causal (both sides of the diagonal)
    (9, 40, True, (10, 0), 8),         # window and chunk together
    (12, 5, True, (-1, -1), 3),        # Sq > Sk: negative diagonal positions
    (6, 50, False, (2, 3), 16),
])
def test_chunk_mask_vs_fp64_brute_force(case):
    Sq, Sk, causal, window, chunk = case
    dt = orc.BF16
    rng = np.random.default_rng(Sq * 1000 + Sk)
    q = rbits(rng, (2, Sq, 4, 128), dt)
    k = rbits(rng, (2, Sk, 2, 128), dt)
    v = rbits(rng, (2, Sk, 2, 128), dt)
    scale = 128 ** -0.5
    out, lse = orc.attention(q, k, v, dtype=dt, scale=scale, causal=causal, window=window, nthreads=NT,
                             chunk=chunk)
    ro, rl = brute.attention_batch(f(q, dt), f(k, dt), f(v, dt), [Sk] * 2, scale, causal, window, chunk=chunk)
    check_vs_brute(out, lse, ro, rl, dt)


def test_chunk_larger_than_everything_is_no_chunk_and_chunk_one_is_the_diagonal():
    dt = orc.FP16
    rng = np.random.default_rng(31)
    q = rbits(rng, (1, 6, 2, 64), dt)
    k = rbits(rng, (1, 20, 2, 64), dt)
    v = rbits(rng, (1, 20, 2, 64), dt)
    a = orc.attention(q, k, v, dtype=dt, scale=0.125, causal=True)
    b = orc.attention(q, k, v, dtype=dt, scale=0.125, causal=True, chunk=1 << 20)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    # chunk 1: query i sees only its diagonal key d = i + 14, so out = v[d] and lse = s[d]
    out, lse = orc.attention(q, k, v, dtype=dt, scale=0.125, causal=False, chunk=1)
    for i in range(6):
        d = i + 14
        assert np.array_equal(out[0, i], v[0, d])
        s = (f(q[0, i], dt).astype(np.float64) * f(k[0, d], dt)).sum(-1) * 0.125
        assert np.allclose(lse[0, :, i], s, rtol=1e-5, atol=1e-5)


def test_append_rotates_at_rotary_seqlens():
    """Token t of batch b lands in slot L_b + t, rotated at P_b + t; P = L is the default."""
    dt = orc.BF16
    rng = np.random.default_rng(32)
    kc = rbits(rng, (2, 24, 2, 128), dt)
    vc = rbits(rng, (2, 24, 2, 128), dt)
    kn = rbits(rng, (2, 3, 2, 128), dt)
    vn = rbits(rng, (2, 3, 2, 128), dt)
    cos, sin = rope_tables(64, 64, dt)
    L = np.array([4, 11], np.int32)
    P = np.array([40, 2], np.int32)
    k2, v2 = orc.kv_append(kc, vc, kn, vn, L, dtype=dt, cos=cos, sin=sin, interleaved=True, rot_pos=P)
    kr = orc.rotary(kn, cos, sin, P, dtype=dt, interleaved=True)
    for b in range(2):
        assert np.array_equal(k2[b, L[b]:L[b] + 3], kr[b])
        assert np.array_equal(v2[b, L[b]:L[b] + 3], vn[b])
        rest = np.ones(24, bool)
        rest[L[b]:L[b] + 3] = False
        assert np.array_equal(k2[b, rest], kc[b, rest])
    k3, _ = orc.kv_append(kc, vc, kn, vn, L, dtype=dt, cos=cos, sin=sin, interleaved=True, rot_pos=L)
    k4, _ = orc.kv_append(kc, vc, kn, vn, L, dtype=dt, cos=cos, sin=sin, interleaved=True)
    assert np.array_equal(k3, k4)


def _dense_case(rng, dt, B=3, Sq=4, cap=96, H=8, Hk=2, s_new=2):
    q = rbits(rng, (B, Sq, H, 128), dt)
    kc = rbits(rng, (B, cap, Hk, 128), dt)
    vc = rbits(rng, (B, cap, Hk, 128), dt)
    kn = rbits(rng, (B, s_new, Hk, 128), dt)
    vn = rbits(rng, (B, s_new, Hk, 128), dt)
    return q, kc, vc, kn, vn


@pytest.mark.parametrize("rot", [False, True])
def test_v3_without_extensions_equals_the_pinned_dense_path(rot):
    dt = orc.BF16
    rng = np.random.default_rng(33)
    q, kc, vc, kn, vn = _dense_case(rng, dt)
    L = np.array([5, 60, 31], np.int32)
    cos, sin = rope_tables(128, 64, dt) if rot else (None, None)
    alibi = (2.0 ** (-8.0 * (np.arange(8) + 1) / 8)).astype(np.float32)
    kw = dict(dtype=dt, cache_seqlens=L, k=kn, v=vn, rotary_cos=cos, rotary_sin=sin, rotary_interleaved=False,
              causal=True, alibi=alibi, cache_batch_idx=np.array([2, 0, 1], np.int32))
    a = orc.kvcache_forward(q, kc, vc, **kw)
    b = orc.kvcache_forward_v3(q, kc, vc, **kw)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_leftpad_drops_the_first_slots():
    """Keys are slots [lp_b, L_b + S_new): garbage before lp_b never reaches the
    output, and the result equals the pinned dense path on a cache whose rows
    are shifted down by lp_b (no rotary: positions do not matter then)."""
    dt = orc.FP16
    rng = np.random.default_rng(34)
    q, kc, vc, kn, vn = _dense_case(rng, dt)
    L = np.array([20, 64, 9], np.int32)
    lp = np.array([7, 0, 9], np.int32)
    kg, vg = kc.copy(), vc.copy()
    for b in range(3):
        kg[b, :lp[b]] = 0x7E00  # NaN
        vg[b, :lp[b]] = 0x7E00
    out, lse, k2, v2 = orc.kvcache_forward_v3(q, kg, vg, dtype=dt, cache_seqlens=L, k=kn, v=vn, causal=True,
                                              window=(12, 0), cache_leftpad=lp)
    assert np.isfinite(f(out, dt)).all()
    ks = np.zeros_like(kc)
    vs = np.zeros_like(vc)
    for b in range(3):
        ks[b, :96 - lp[b]] = kc[b, lp[b]:]
        vs[b, :96 - lp[b]] = vc[b, lp[b]:]
    o2, l2, k3, _ = orc.kvcache_forward(q, ks, vs, dtype=dt, cache_seqlens=L - lp, k=kn, v=vn, causal=True,
                                        window=(12, 0))
    assert np.array_equal(out, o2) and np.array_equal(lse, l2)
    for b in range(3):  # the append still lands at slot L_b
        assert np.array_equal(k2[b, L[b]:L[b] + 2], kn[b])


def test_leftpad_equal_to_seqlens_sees_only_the_new_token():
    dt = orc.BF16
    rng = np.random.default_rng(35)
    q, kc, vc, kn, vn = _dense_case(rng, dt, s_new=1, Sq=1)
    L = np.array([10, 50, 3], np.int32)
    out, lse, _, _ = orc.kvcache_forward_v3(q, kc, vc, dtype=dt, cache_seqlens=L, k=kn, v=vn, causal=True,
                                            cache_leftpad=L)
    for b in range(3):
        for h in range(8):
            assert np.array_equal(out[b, 0, h], vn[b, 0, h // 4])
            s = (f(q[b, 0, h], dt).astype(np.float64) * f(kn[b, 0, h // 4], dt)).sum() * 128 ** -0.5
            assert abs(lse[b, h, 0] - s) <= 1e-5 * max(1.0, abs(s))


@pytest.mark.parametrize("paged", [False, True])
def test_ragged_q_and_new_tokens_equal_the_dense_layout(paged):
    """Equal lengths in the ragged layouts give exactly the dense result."""
    dt = orc.BF16
    rng = np.random.default_rng(36)
    B, Sq, s_new, page = 3, 5, 3, 16
    q, kc, vc, kn, vn = _dense_case(rng, dt, B=B, Sq=Sq, s_new=s_new)
    L = np.array([2, 70, 40], np.int32)
    cos, sin = rope_tables(128, 32, dt)
    bt = None
    if paged:
        nb = B * 96 // page
        perm = rng.permutation(nb).astype(np.int32)
        bt = perm.reshape(B, 96 // page)
        kp = np.zeros((nb, page) + kc.shape[2:], np.uint16)
        vp = np.zeros_like(kp)
        for b in range(B):
            for j in range(96):
                kp[bt[b, j // page], j % page] = kc[b, j]
                vp[bt[b, j // page], j % page] = vc[b, j]
        kc, vc = kp, vp
    kw = dict(dtype=dt, cache_seqlens=L, rotary_cos=cos, rotary_sin=sin, causal=True, block_table=bt,
              rotary_seqlens=np.array([9, 3, 100], np.int32), attention_chunk=32)
    a = orc.kvcache_forward_v3(q, kc, vc, k=kn, v=vn, **kw)
    cu_q = np.arange(B + 1, dtype=np.int32) * Sq
    cu_n = np.arange(B + 1, dtype=np.int32) * s_new
    b = orc.kvcache_forward_v3(q.reshape(B * Sq, 8, 128), kc, vc, k=kn.reshape(B * s_new, 2, 128),
                               v=vn.reshape(B * s_new, 2, 128), cu_seqlens_q=cu_q, max_seqlen_q=Sq,
                               cu_seqlens_k_new=cu_n, **kw)
    assert np.array_equal(a[0].reshape(B * Sq, 8, 128), b[0])
    assert np.array_equal(a[1].transpose(1, 0, 2).reshape(8, B * Sq), b[1])
    assert np.array_equal(a[2], b[2]) and np.array_equal(a[3], b[3])


def test_ragged_sequences_vs_fp64_brute_force():
    """Different query and new-token counts per sequence, with rotary at
    rotary_seqlens, checked against append + rotate + brute force."""
    dt = orc.BF16
    rng = np.random.default_rng(37)
    B, H, Hk, cap = 3, 4, 2, 64
    nq, nn = [3, 1, 6], [2, 0, 4]
    L = np.array([10, 33, 0], np.int32)
    P = np.array([5, 40, 7], np.int32)
    cu_q = np.concatenate([[0], np.cumsum(nq)]).astype(np.int32)
    cu_n = np.concatenate([[0], np.cumsum(nn)]).astype(np.int32)
    q = rbits(rng, (cu_q[-1], H, 128), dt)
    kn = rbits(rng, (cu_n[-1], Hk, 128), dt)
    vn = rbits(rng, (cu_n[-1], Hk, 128), dt)
    kc = rbits(rng, (B, cap, Hk, 128), dt)
    vc = rbits(rng, (B, cap, Hk, 128), dt)
    cos, sin = rope_tables(128, 128, dt)
    out, lse, k2, v2 = orc.kvcache_forward_v3(q, kc, vc, dtype=dt, cache_seqlens=L, k=kn, v=vn, rotary_cos=cos,
                                              rotary_sin=sin, rotary_interleaved=True, causal=True,
                                              cu_seqlens_q=cu_q, max_seqlen_q=6, cu_seqlens_k_new=cu_n,
                                              rotary_seqlens=P)
    for b in range(B):
        knb = kn[cu_n[b]:cu_n[b + 1]]
        if nn[b]:
            kr = orc.rotary(knb[None], cos, sin, P[b:b + 1], dtype=dt, interleaved=True)[0]
            assert np.array_equal(k2[b, L[b]:L[b] + nn[b]], kr)
            assert np.array_equal(v2[b, L[b]:L[b] + nn[b]], vn[cu_n[b]:cu_n[b + 1]])
        qb = orc.rotary(q[cu_q[b]:cu_q[b + 1]][None], cos, sin, P[b:b + 1], dtype=dt, interleaved=True)[0]
        n = L[b] + nn[b]
        ro, rl = brute.attention(f(qb, dt), f(k2[b, :n], dt), f(v2[b, :n], dt), 128 ** -0.5, causal=True)
        got = f(out[cu_q[b]:cu_q[b + 1]], dt)
        assert np.abs(got - ro).max() <= 1e-2
        assert np.allclose(lse[:, cu_q[b]:cu_q[b + 1]], rl, rtol=2e-5)
