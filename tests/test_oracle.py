"""Pins the CPU oracle (oracle/fa_oracle.c) before it is trusted as the checker.

Each test checks the oracle against something it does not share code with:
the float64 brute force in tests/golden/brute.py (one-pass softmax over a
mask built from triangular matrices), closed forms, the README's mask
diagrams, library routines (numpy/torch dtype conversions, numpy fancy
indexing, torch's textbook rotary formulation) or invariances that a wrong
index, sign or dropped term would break. CPU only.
"""
import os

import numpy as np
import pytest
import torch

from oracle import fa_oracle as orc
from tests._util import LSE_ATOL
from tests.golden import brute

NT = min(8, os.cpu_count() or 1)
TOL = {orc.FP16: 2e-3, orc.BF16: 1e-2}


def rbits(rng, shape, dtype, scale=1.0):
    return orc.to_bits(rng.standard_normal(shape).astype(np.float32) * scale, dtype)


def f(bits, dtype):
    return orc.from_bits(bits, dtype).reshape(bits.shape)


def check_vs_brute(out, lse, ref_out, ref_lse, dtype, lse_rtol=2e-5):
    got = f(out, dtype)
    assert np.abs(got - ref_out).max() <= TOL[dtype], np.abs(got - ref_out).max()
    inf = np.isinf(ref_lse)
    assert np.array_equal(np.isinf(lse), inf)
    if (~inf).any():
        err = np.abs(lse[~inf].astype(np.float64) - ref_lse[~inf])
        assert (err <= lse_rtol * np.abs(ref_lse[~inf]) + LSE_ATOL).all(), err.max()
    assert np.all(got[np.isinf(ref_lse).transpose(0, 2, 1)] == 0)


CASES = [
    # B, Sq, Sk, H, Hk, dtype, causal, window, alibi, softcap
    (2, 16, 16, 4, 4, orc.FP16, True, (-1, -1), False, 0.0),
    (2, 9, 700, 4, 2, orc.BF16, True, (-1, -1), False, 0.0),       # two key stacks, GQA
    (1, 5, 1100, 8, 1, orc.FP16, False, (-1, -1), False, 0.0),     # three stacks, MQA
    (2, 12, 5, 4, 2, orc.FP16, True, (-1, -1), False, 0.0),        # Sq > Sk: empty rows
    (2, 7, 600, 4, 4, orc.BF16, True, (100, 0), False, 0.0),       # sliding window
    (1, 8, 40, 4, 2, orc.FP16, False, (3, 2), False, 0.0),         # two-sided window
    (2, 4, 530, 8, 2, orc.BF16, True, (-1, -1), True, 0.0),        # ALiBi
    (1, 6, 64, 4, 4, orc.FP16, False, (-1, -1), False, 5.0),       # softcap
    (2, 3, 900, 4, 1, orc.BF16, True, (300, 0), True, 8.0),        # everything at once
]


@pytest.mark.parametrize("case", CASES, ids=[str(i) for i in range(len(CASES))])
def test_attention_vs_fp64_brute_force(case):
    B, Sq, Sk, H, Hk, dt, causal, window, use_alibi, softcap = case
    rng = np.random.default_rng(hash(case) & 0xFFFF)
    q = rbits(rng, (B, Sq, H, 128), dt)
    k = rbits(rng, (B, Sk, Hk, 128), dt)
    v = rbits(rng, (B, Sk, Hk, 128), dt)
    scale = 128 ** -0.5
    alibi = (2.0 ** (-8.0 * (np.arange(H) + 1) / H)).astype(np.float32) if use_alibi else None
    out, lse = orc.attention(q, k, v, dtype=dt, scale=scale, causal=causal, window=window, alibi=alibi,
                             softcap=softcap, nthreads=NT)
    ro, rl = brute.attention_batch(f(q, dt), f(k, dt), f(v, dt), [Sk] * B, scale, causal, window, alibi, softcap)
    check_vs_brute(out, lse, ro, rl, dt)


def test_varlen_and_seqlens_vs_brute_force():
    dt = orc.BF16
    rng = np.random.default_rng(3)
    lens_q = [3, 1, 7]
    lens_k = [40, 600, 9]
    H, Hk = 4, 2
    cu_q = np.cumsum([0] + lens_q).astype(np.int32)
    cu_k = np.cumsum([0] + lens_k).astype(np.int32)
    q = rbits(rng, (cu_q[-1], H, 128), dt)
    k = rbits(rng, (cu_k[-1], Hk, 128), dt)
    v = rbits(rng, (cu_k[-1], Hk, 128), dt)
    out, lse = orc.attention(q, k, v, dtype=dt, scale=0.1, causal=True, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                             nthreads=NT)
    for b in range(3):
        qs, ks = slice(cu_q[b], cu_q[b + 1]), slice(cu_k[b], cu_k[b + 1])
        ro, rl = brute.attention(f(q[qs], dt), f(k[ks], dt), f(v[ks], dt), 0.1, causal=True)
        got = f(out[qs], dt)
        assert np.abs(got - ro).max() <= TOL[dt]
        np.testing.assert_allclose(lse[:, qs], rl, rtol=2e-5)


# ---- closed forms ------------------------------------------------------------------

@pytest.mark.parametrize("dt", [orc.FP16, orc.BF16])
def test_single_key_returns_v(dt):
    """Sk = 1: the softmax weight is exactly 1, so out = v bit for bit and lse = s."""
    rng = np.random.default_rng(5)
    q = rbits(rng, (2, 1, 4, 128), dt)
    k = rbits(rng, (2, 1, 2, 128), dt)
    v = rbits(rng, (2, 1, 2, 128), dt)
    out, lse = orc.attention(q, k, v, dtype=dt, scale=0.25, causal=True)
    for h in range(4):
        assert np.array_equal(out[:, 0, h], v[:, 0, h // 2])
        s = (f(q, dt)[:, 0, h].astype(np.float64) * f(k, dt)[:, 0, h // 2]).sum(-1) * 0.25
        np.testing.assert_allclose(lse[:, h, 0], s, rtol=1e-6, atol=1e-6)


def test_identical_keys_mean_and_log_n():
    """All keys equal: uniform weights, out = mean(v), lse = s + ln(n)."""
    dt = orc.FP16
    rng = np.random.default_rng(6)
    n = 1000
    q = rbits(rng, (1, 1, 2, 128), dt)
    k1 = rbits(rng, (1, 1, 1, 128), dt)
    k = np.repeat(k1, n, axis=1)
    v = rbits(rng, (1, n, 1, 128), dt)
    out, lse = orc.attention(q, k, v, dtype=dt, scale=0.05)
    vm = f(v, dt)[0, :, 0].astype(np.float64).mean(0)
    for h in range(2):
        assert np.abs(f(out, dt)[0, 0, h] - vm).max() < 1e-3
        s = float((f(q, dt)[0, 0, h].astype(np.float64) * f(k1, dt)[0, 0, 0]).sum() * 0.05)
        assert abs(lse[0, h, 0] - (s + np.log(n))) < 1e-5


@pytest.mark.parametrize("dt", [orc.FP16, orc.BF16])
def test_p_rounded_to_dtype_before_pv(dt):
    """The golden casts P to the input dtype before P.V but sums the fp32 P
    (tests/test_flash_attn_npu_v3.py:127-131 in the reference). Key 0 scores 0
    (P = 1) with v = -50; 100 keys score s with v = 1, where exp(s) is not 0.5
    in fp32 but rounds to exactly 0.5 in the dtype (bf16: s = -0.69140625,
    P = 0.50085; fp16: s = -0.693359375, P = 0.49989). With P rounded the P.V
    sum is -50 + 100 * 0.5 = 0 exactly; unrounded it is +0.085 / -0.011."""
    n = 100
    s = -0.69140625 if dt == orc.BF16 else -0.693359375
    q = np.zeros((1, 1, 1, 128), np.float32)
    q[..., 0] = 1.0
    k = np.zeros((1, n + 1, 1, 128), np.float32)
    k[0, 1:, 0, 0] = s
    v = np.zeros((1, n + 1, 1, 128), np.float32)
    v[0, 0, 0, :] = -50.0
    v[0, 1:, 0, :] = 1.0
    out, lse = orc.attention(orc.to_bits(q, dt), orc.to_bits(k, dt), orc.to_bits(v, dt), dtype=dt, scale=1.0)
    assert np.all(f(out, dt) == 0.0)
    p = np.exp(np.float32(s))
    assert p != 0.5 and f(orc.to_bits(np.float32(p), dt), dt) == 0.5
    # the row sum (and so the LSE) uses the unrounded P
    assert abs(lse[0, 0, 0] - np.log(1.0 + n * float(p))) < 1e-5


# ---- masks ---------------------------------------------------------------------------

def visible_by_onehot(sq, sk, causal, window):
    """Returns the (sq, sk) 0/1 visibility read back from the oracle: q = 0 gives
    uniform weights over the visible keys and v[j] = e_j, so out[i, j] > 0 iff key j
    is visible to query i; lse = +inf marks an empty row."""
    dt = orc.FP16
    q = np.zeros((1, sq, 1, 128), np.float32)
    k = np.zeros((1, sk, 1, 128), np.float32)
    v = np.zeros((1, sk, 1, 128), np.float32)
    for j in range(sk):
        v[0, j, 0, j] = 1.0
    out, lse = orc.attention(orc.to_bits(q, dt), orc.to_bits(k, dt), orc.to_bits(v, dt), dtype=dt, scale=1.0,
                             causal=causal, window=window)
    o = f(out, dt)[0, :, 0, :sk]
    vis = (o > 0).astype(int)
    for i in range(sq):
        nv = vis[i].sum()
        if nv:
            np.testing.assert_array_equal(o[i][vis[i] == 1], np.float16(1.0 / nv).astype(np.float32))
            assert np.isfinite(lse[0, 0, i])
        else:
            assert np.isinf(lse[0, 0, i]) and lse[0, 0, i] > 0
    return vis


def test_readme_causal_masks():
    """The two bottom-right causal masks drawn in the reference README (README.md:116-126)."""
    np.testing.assert_array_equal(visible_by_onehot(2, 5, True, (-1, -1)),
                                  [[1, 1, 1, 1, 0],
                                   [1, 1, 1, 1, 1]])
    np.testing.assert_array_equal(visible_by_onehot(5, 2, True, (-1, -1)),
                                  [[0, 0], [0, 0], [0, 0], [1, 0], [1, 1]])


def test_readme_window_rule():
    """Query i sees keys [i + Sk - Sq - wl, i + Sk - Sq + wr] (README.md:128-130)."""
    sq, sk, wl, wr = 4, 9, 2, 1
    exp = np.zeros((sq, sk), int)
    for i in range(sq):
        for j in range(sk):
            exp[i, j] = int(i + sk - sq - wl <= j <= i + sk - sq + wr)
    np.testing.assert_array_equal(visible_by_onehot(sq, sk, False, (wl, wr)), exp)
    # causal forces wr = 0
    exp_c = np.array([[int(i + sk - sq - wl <= j <= i + sk - sq) for j in range(sk)] for i in range(sq)])
    np.testing.assert_array_equal(visible_by_onehot(sq, sk, True, (wl, wr)), exp_c)


@pytest.mark.parametrize("sq,sk,causal,wl,wr", [
    (1, 10, True, -1, -1), (5, 5, False, 4, 4), (3, 8, True, 7, 5), (6, 3, False, 1, -1), (4, 12, False, 3, 0),
])
def test_masks_match_triangular_construction(sq, sk, causal, wl, wr):
    np.testing.assert_array_equal(visible_by_onehot(sq, sk, causal, (wl, wr)),
                                  brute.mask_keep(sq, sk, causal, (wl, wr)).astype(int))


def test_window_normalisation_known_answers():
    """tests/fa_small_op_golden.py:21-32 in the reference, worked by hand."""
    assert orc.normalize_window(1, 100, True, -1, -1) == (-1, 0)
    assert orc.normalize_window(128, 128, False, 127, 127) == (-1, -1)
    assert orc.normalize_window(128, 128, False, 126, 126) == (126, 126)
    assert orc.normalize_window(4, 4096, True, 4096, 0) == (-1, 0)
    assert orc.normalize_window(4, 65536, True, 4096, 0) == (4096, 0)
    assert brute.normalize_window(4, 65536, True, 4096, 0) == (4096, 0, False, True)
    assert brute.normalize_window(8, 8, True, -1, 5) == (-1, 0, True, False)


# ---- layout invariances ------------------------------------------------------------------

def test_gqa_equals_mha_with_repeated_kv():
    """q head h reads kv head h // (H/Hk): the same as MHA on repeat_interleave'd K/V
    (broadcast_kv_single, tests/fa_small_op_golden.py:11-18), bit for bit."""
    dt = orc.BF16
    rng = np.random.default_rng(8)
    q = rbits(rng, (2, 5, 8, 128), dt)
    k = rbits(rng, (2, 77, 2, 128), dt)
    v = rbits(rng, (2, 77, 2, 128), dt)
    o1, l1 = orc.attention(q, k, v, dtype=dt, scale=0.09, causal=True)
    o2, l2 = orc.attention(q, np.repeat(k, 4, axis=2), np.repeat(v, 4, axis=2), dtype=dt, scale=0.09, causal=True)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


def _paged(rng, kc, page, seqlens):
    """Scatter a contiguous cache (B, S, Hk, D) into a shuffled block pool."""
    B, S, Hk, D = kc.shape
    nb = (S + page - 1) // page
    perm = rng.permutation(B * nb + 3)
    pool = np.zeros((B * nb + 3, page, Hk, D), np.uint16)
    bt = np.zeros((B, nb), np.int32)
    for b in range(B):
        for i in range(nb):
            blk = perm[b * nb + i]
            bt[b, i] = blk
            seg = kc[b, i * page:(i + 1) * page]
            pool[blk, :seg.shape[0]] = seg
    return pool, bt


def test_paged_equals_contiguous_bitwise():
    dt = orc.BF16
    rng = np.random.default_rng(9)
    B, S, page = 3, 96, 16
    q = rbits(rng, (B, 2, 4, 128), dt)
    kc = rbits(rng, (B, S, 2, 128), dt)
    vc = rbits(rng, (B, S, 2, 128), dt)
    sl = np.array([96, 17, 50], np.int32)
    o1, l1 = orc.attention(q, kc, vc, dtype=dt, scale=0.1, causal=True, seqlens_k=sl)
    kp, bt = _paged(np.random.default_rng(1), kc, page, sl)
    vp, _ = _paged(np.random.default_rng(1), vc, page, sl)
    o2, l2 = orc.attention(q, kp, vp, dtype=dt, scale=0.1, causal=True, seqlens_k=sl, block_table=bt)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


def test_cache_batch_idx_selects_rows():
    dt = orc.FP16
    rng = np.random.default_rng(10)
    q = rbits(rng, (3, 1, 2, 128), dt)
    kc = rbits(rng, (5, 40, 1, 128), dt)
    vc = rbits(rng, (5, 40, 1, 128), dt)
    idx = np.array([4, 0, 2], np.int32)
    sl = np.array([40, 7, 23], np.int32)
    o1, l1 = orc.attention(q, kc, vc, dtype=dt, scale=0.1, seqlens_k=sl, batch_idx=idx)
    o2, l2 = orc.attention(q, kc[idx], vc[idx], dtype=dt, scale=0.1, seqlens_k=sl)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


def test_paged_with_cache_batch_idx_selects_block_table_rows():
    """cache_batch_idx with a block table picks block-table row idx[b] (the
    build's definition for config 5), while cache_seqlens stay indexed by b."""
    dt = orc.BF16
    rng = np.random.default_rng(24)
    B, S, page = 4, 64, 16
    q = rbits(rng, (3, 1, 2, 128), dt)
    kc = rbits(rng, (B, S, 1, 128), dt)
    vc = rbits(rng, (B, S, 1, 128), dt)
    idx = np.array([2, 3, 0], np.int32)
    sl = np.array([64, 20, 33], np.int32)
    kp, bt = _paged(np.random.default_rng(2), kc, page, sl)
    vp, _ = _paged(np.random.default_rng(2), vc, page, sl)
    o1, l1 = orc.attention(q, kp, vp, dtype=dt, scale=0.1, seqlens_k=sl, block_table=bt, batch_idx=idx)
    o2, l2 = orc.attention(q, kc[idx], vc[idx], dtype=dt, scale=0.1, seqlens_k=sl)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


def test_varlen_equals_padded_batch():
    dt = orc.BF16
    rng = np.random.default_rng(11)
    q = rbits(rng, (2, 6, 4, 128), dt)
    k = rbits(rng, (2, 30, 2, 128), dt)
    v = rbits(rng, (2, 30, 2, 128), dt)
    o1, l1 = orc.attention(q, k, v, dtype=dt, scale=0.1, causal=True)
    cu = np.array([0, 6, 12], np.int32)
    cuk = np.array([0, 30, 60], np.int32)
    o2, l2 = orc.attention(q.reshape(12, 4, 128), k.reshape(60, 2, 128), v.reshape(60, 2, 128), dtype=dt, scale=0.1,
                           causal=True, cu_seqlens_q=cu, cu_seqlens_k=cuk)
    assert np.array_equal(o1.reshape(12, 4, 128), o2)
    assert np.array_equal(l1.transpose(1, 0, 2).reshape(4, 12), l2)


def test_alibi_zero_slopes_is_no_alibi_and_batch_broadcast():
    dt = orc.BF16
    rng = np.random.default_rng(12)
    q = rbits(rng, (2, 3, 4, 128), dt)
    k = rbits(rng, (2, 50, 2, 128), dt)
    v = rbits(rng, (2, 50, 2, 128), dt)
    o0, l0 = orc.attention(q, k, v, dtype=dt, scale=0.1, causal=True)
    o1, l1 = orc.attention(q, k, v, dtype=dt, scale=0.1, causal=True, alibi=np.zeros(4, np.float32))
    assert np.array_equal(o0, o1) and np.array_equal(l0, l1)
    sl = np.array([0.5, 0.25, 0.125, 0.0625], np.float32)
    o2, l2 = orc.attention(q, k, v, dtype=dt, scale=0.1, causal=True, alibi=sl)
    o3, l3 = orc.attention(q, k, v, dtype=dt, scale=0.1, causal=True, alibi=np.stack([sl, sl]))
    assert np.array_equal(o2, o3) and np.array_equal(l2, l3)
    assert not np.array_equal(o0, o2)


# ---- rotary ----------------------------------------------------------------------------------

def rope_tables(n, rd, dt, base=10000.0):
    inv = 1.0 / base ** (np.arange(0, rd, 2, dtype=np.float64) / rd)
    ang = np.outer(np.arange(n), inv)
    return orc.to_bits(np.cos(ang).astype(np.float32), dt), orc.to_bits(np.sin(ang).astype(np.float32), dt)


def torch_rotary(x, cos, sin, interleaved):
    """The textbook formulation x * cos + rotate_half(x) * sin in fp32 (the
    `apply_rotary_emb_torch` form the flash-attention API documents), on
    x (S, H, rd) and cos/sin (S, rd/2)."""
    if interleaved:
        cos = torch.repeat_interleave(cos, 2, dim=-1)
        sin = torch.repeat_interleave(sin, 2, dim=-1)
        x1, x2 = x[..., ::2], x[..., 1::2]
        rot = torch.stack((-x2, x1), dim=-1).flatten(-2)
    else:
        cos = torch.cat([cos, cos], dim=-1)
        sin = torch.cat([sin, sin], dim=-1)
        x1, x2 = x.chunk(2, dim=-1)
        rot = torch.cat((-x2, x1), dim=-1)
    return x * cos[:, None, :] + rot * sin[:, None, :]


@pytest.mark.parametrize("interleaved", [True, False])
@pytest.mark.parametrize("dt", [orc.FP16, orc.BF16])
@pytest.mark.parametrize("rd", [128, 64])
def test_rotary_matches_textbook_formulation(interleaved, dt, rd):
    rng = np.random.default_rng(13)
    B, S, H = 2, 5, 3
    x = rbits(rng, (B, S, H, 128), dt)
    cos, sin = rope_tables(64, rd, dt)
    L = np.array([0, 37], np.int32)
    y = orc.rotary(x, cos, sin, L, dtype=dt, interleaved=interleaved)
    tdt = torch.float16 if dt == orc.FP16 else torch.bfloat16
    for b in range(B):
        pos = L[b] + np.arange(S)
        xt = torch.from_numpy(f(x[b], dt)[..., :rd].copy())
        ct = torch.from_numpy(f(cos[pos], dt).copy())
        st = torch.from_numpy(f(sin[pos], dt).copy())
        ref = torch_rotary(xt, ct, st, interleaved).to(tdt).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(y[b, ..., :rd], ref)
        assert np.array_equal(y[b, ..., rd:], x[b, ..., rd:])  # dims >= rotary_dim untouched


def test_rotary_identity_same_pos_and_norm():
    dt = orc.BF16
    rng = np.random.default_rng(14)
    x = rbits(rng, (1, 4, 2, 128), dt)
    one = orc.to_bits(np.ones((8, 64), np.float32), dt)
    zero = orc.to_bits(np.zeros((8, 64), np.float32), dt)
    assert np.array_equal(orc.rotary(x, one, zero, [0], dtype=dt, interleaved=False), x)
    cos, sin = rope_tables(16, 128, dt)
    # same_pos: every row rotated at position seqlens[b]
    y = orc.rotary(x, cos, sin, [5], dtype=dt, interleaved=True, same_pos=True)
    for i in range(4):
        xi = np.repeat(x[:, i:i + 1], 4, axis=1)
        assert np.array_equal(y[:, i], orc.rotary(xi, cos, sin, [5], dtype=dt, interleaved=True, same_pos=True)[:, 0])
    # a rotation keeps the norm (to the dtype's rounding)
    nx = np.linalg.norm(f(x, dt), axis=-1)
    ny = np.linalg.norm(f(y, dt), axis=-1)
    np.testing.assert_allclose(nx, ny, rtol=2e-2)


def test_rotary_vs_complex_rotation():
    """Interleaved pairs are complex numbers multiplied by e^{i*pos*theta_k}."""
    dt = orc.FP16
    rng = np.random.default_rng(15)
    x = rbits(rng, (1, 3, 1, 128), dt)
    cos, sin = rope_tables(8, 128, dt)
    y = orc.rotary(x, cos, sin, [2], dtype=dt, interleaved=True)
    xf = f(x, dt)[0, :, 0].astype(np.float64)
    z = xf[:, 0::2] + 1j * xf[:, 1::2]
    rot = f(cos, dt)[2:5].astype(np.float64) + 1j * f(sin, dt)[2:5]
    zr = z * rot
    yf = f(y, dt)[0, :, 0]
    np.testing.assert_allclose(yf[:, 0::2], zr.real, atol=8e-3)
    np.testing.assert_allclose(yf[:, 1::2], zr.imag, atol=8e-3)


# ---- append ----------------------------------------------------------------------------------

def test_append_contiguous_and_batch_idx_vs_fancy_indexing():
    dt = orc.BF16
    rng = np.random.default_rng(16)
    kc = rbits(rng, (4, 32, 2, 128), dt)
    vc = rbits(rng, (4, 32, 2, 128), dt)
    kn = rbits(rng, (3, 3, 2, 128), dt)
    vn = rbits(rng, (3, 3, 2, 128), dt)
    L = np.array([0, 10, 29], np.int32)
    idx = np.array([2, 0, 3], np.int32)
    k2, v2 = orc.kv_append(kc, vc, kn, vn, L, dtype=dt, batch_idx=idx)
    ek, ev = kc.copy(), vc.copy()
    for b in range(3):
        ek[idx[b], L[b]:L[b] + 3] = kn[b]
        ev[idx[b], L[b]:L[b] + 3] = vn[b]
    assert np.array_equal(k2, ek) and np.array_equal(v2, ev)
    assert np.array_equal(k2[1], kc[1])  # untouched row


def test_append_paged_vs_fancy_indexing():
    dt = orc.FP16
    rng = np.random.default_rng(17)
    page = 8
    pool_k = rbits(rng, (10, page, 1, 128), dt)
    pool_v = rbits(rng, (10, page, 1, 128), dt)
    bt = np.array([[7, 2, 9], [0, 5, 1]], np.int32)
    kn = rbits(rng, (2, 4, 1, 128), dt)
    vn = rbits(rng, (2, 4, 1, 128), dt)
    L = np.array([6, 13], np.int32)
    k2, v2 = orc.kv_append(pool_k, pool_v, kn, vn, L, dtype=dt, block_table=bt)
    ek, ev = pool_k.copy(), pool_v.copy()
    for b in range(2):
        for t in range(4):
            j = L[b] + t
            ek[bt[b, j // page], j % page] = kn[b, t]
            ev[bt[b, j // page], j % page] = vn[b, t]
    assert np.array_equal(k2, ek) and np.array_equal(v2, ev)


def test_append_with_rotary_writes_rotated_k():
    dt = orc.BF16
    rng = np.random.default_rng(18)
    kc = rbits(rng, (2, 16, 2, 128), dt)
    vc = rbits(rng, (2, 16, 2, 128), dt)
    kn = rbits(rng, (2, 2, 2, 128), dt)
    vn = rbits(rng, (2, 2, 2, 128), dt)
    cos, sin = rope_tables(16, 64, dt)
    L = np.array([3, 9], np.int32)
    k2, v2 = orc.kv_append(kc, vc, kn, vn, L, dtype=dt, cos=cos, sin=sin, interleaved=False)
    kr = orc.rotary(kn, cos, sin, L, dtype=dt, interleaved=False)
    for b in range(2):
        assert np.array_equal(k2[b, L[b]:L[b] + 2], kr[b])
        assert np.array_equal(v2[b, L[b]:L[b] + 2], vn[b])  # v is never rotated


def test_kvcache_forward_is_append_then_attention():
    dt = orc.BF16
    rng = np.random.default_rng(19)
    q = rbits(rng, (2, 2, 4, 128), dt)
    kc = rbits(rng, (2, 64, 2, 128), dt)
    vc = rbits(rng, (2, 64, 2, 128), dt)
    kn = rbits(rng, (2, 2, 2, 128), dt)
    vn = rbits(rng, (2, 2, 2, 128), dt)
    L = np.array([5, 40], np.int32)
    out, lse, k2, v2 = orc.kvcache_forward(q, kc, vc, dtype=dt, cache_seqlens=L, k=kn, v=vn, causal=True)
    ro, rl = brute.attention_batch(f(q, dt), f(k2, dt), f(v2, dt), L + 2, 128 ** -0.5, causal=True)
    check_vs_brute(out, lse, ro, rl, dt)


# ---- split-KV combine --------------------------------------------------------------------------

def test_combine_equals_full_softmax():
    """Attention over disjoint key ranges, merged by LSE, equals attention over
    all keys (the closed-form merge of CombineScale.hpp:150-194)."""
    rng = np.random.default_rng(20)
    q = rng.standard_normal((3, 2, 64))
    k = rng.standard_normal((90, 1, 64))
    v = rng.standard_normal((90, 1, 64))
    full_o, full_l = brute.attention(q, k, v, 0.125)
    cuts = [0, 10, 55, 90]
    parts = [brute.attention(q, k[a:b], v[a:b], 0.125) for a, b in zip(cuts[:-1], cuts[1:])]
    # rows r = (head, query): (S, R, Dv) / (S, R)
    op = np.stack([p[0].transpose(1, 0, 2).reshape(6, 64) for p in parts]).astype(np.float32)
    lp = np.stack([p[1].reshape(6) for p in parts]).astype(np.float32)
    o, l = orc.combine(op, lp)
    np.testing.assert_allclose(o, full_o.transpose(1, 0, 2).reshape(6, 64), atol=2e-6)
    np.testing.assert_allclose(l, full_l.reshape(6), rtol=1e-6)


def test_combine_ignores_empty_splits():
    rng = np.random.default_rng(21)
    op = rng.standard_normal((3, 4, 16)).astype(np.float32)
    lp = rng.standard_normal((3, 4)).astype(np.float32)
    lp[1, :] = np.inf        # split that saw no visible key (the +inf convention)
    lp[2, 2] = -np.inf
    o, l = orc.combine(op, lp)
    o2, l2 = orc.combine(op[[0, 2]], np.stack([lp[0], np.where(np.isfinite(lp[2]), lp[2], -np.inf)]))
    np.testing.assert_allclose(o, o2, rtol=1e-6)
    np.testing.assert_allclose(l, l2, rtol=1e-6)
    np.testing.assert_array_equal(o[2], op[0, 2])  # only split 0 is finite for row 2
    lp[:] = np.inf
    o, l = orc.combine(op, lp)
    assert np.all(o == 0) and np.all(np.isinf(l))


# ---- 16-bit conversions --------------------------------------------------------------------------

def test_fp16_conversions_vs_numpy():
    L = orc.lib()
    allh = np.arange(65536, dtype=np.uint16)
    ref = allh.view(np.float16).astype(np.float32)
    got = np.array([L.orc_f16_to_f32(int(h)) for h in allh[::7]], np.float32)
    r = ref[::7]
    assert np.array_equal(np.isnan(got), np.isnan(r))
    assert np.array_equal(got[~np.isnan(r)], r[~np.isnan(r)])
    rng = np.random.default_rng(22)
    xs = np.concatenate([rng.standard_normal(3000).astype(np.float32) * 10.0 ** rng.integers(-8, 5, 3000),
                         np.array([65504, 65520, 1e6, -1e6, 6e-8, 3e-8, 2.9e-8, 0.0, -0.0], np.float32),
                         (np.arange(2048, dtype=np.float32) + 0.5) / 1024])  # ties
    got = np.array([L.orc_f32_to_f16(float(x)) for x in xs], np.uint16)
    with np.errstate(over="ignore"):
        ref = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_bf16_conversions_vs_torch():
    L = orc.lib()
    allb = np.arange(0, 65536, 5, dtype=np.uint16)
    ref = torch.from_numpy(allb.view(np.int16)).view(torch.bfloat16).float().numpy()
    got = np.array([L.orc_bf16_to_f32(int(h)) for h in allb], np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(ref)], ref[~np.isnan(ref)])
    rng = np.random.default_rng(23)
    xs = np.concatenate([rng.standard_normal(3000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 3000),
                         (np.arange(1, 600, dtype=np.uint32) << 15 | 0x3F800000).view(np.float32)])  # ties
    got = np.array([L.orc_f32_to_bf16(float(x)) for x in xs], np.uint16)
    ref = torch.from_numpy(xs).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    assert np.array_equal(orc.to_bits(xs, orc.BF16), ref)


# ---- qv (FlashAttention-3: scores = q.k + qv.v) --------------------------------------------
@pytest.mark.parametrize("dt,softcap,alibi", [(orc.FP16, 0.0, False), (orc.BF16, 0.0, False),
                                               (orc.BF16, 4.0, False), (orc.FP16, 0.0, True)])
def test_qv_is_attention_over_concatenated_head_dims(dt, softcap, alibi):
    # the oracle accumulates q.k then qv.v in one fp32 sum, before the scale,
    # the soft cap and the ALiBi bias: the same bits as [q, qv] . [k, v] over
    # the concatenated head dims
    rng = np.random.default_rng(71)
    B, Sq, Sk, H, Hk, D = 2, 3, 600, 8, 2, 64
    q, qv = rbits(rng, (B, Sq, H, D), dt), rbits(rng, (B, Sq, H, D), dt)
    k, v = rbits(rng, (B, Sk, Hk, D), dt), rbits(rng, (B, Sk, Hk, D), dt)
    scale = (2 * D) ** -0.5
    sl = (2.0 ** (-8.0 * (np.arange(H) + 1) / H)).astype(np.float32) if alibi else None
    o1, l1 = orc.attention(q, k, v, dtype=dt, scale=scale, causal=True, qv=qv, softcap=softcap, alibi=sl,
                           nthreads=NT)
    o2, l2 = orc.attention(np.concatenate([q, qv], -1), np.concatenate([k, v], -1), v, dtype=dt, scale=scale,
                           causal=True, softcap=softcap, alibi=sl, nthreads=NT)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


def test_qv_vs_fp64_brute_force():
    rng = np.random.default_rng(72)
    dt = orc.BF16
    B, Sq, Sk, H, Hk, D = 2, 4, 530, 8, 2, 128
    q, qv = rbits(rng, (B, Sq, H, D), dt), rbits(rng, (B, Sq, H, D), dt)
    k, v = rbits(rng, (B, Sk, Hk, D), dt), rbits(rng, (B, Sk, Hk, D), dt)
    scale = (2 * D) ** -0.5
    out, lse = orc.attention(q, k, v, dtype=dt, scale=scale, causal=True, window=(200, 0), qv=qv, nthreads=NT)
    qf, qvf, kf, vf = f(q, dt), f(qv, dt), f(k, dt), f(v, dt)
    ro, rl = brute.attention_batch(np.concatenate([qf, qvf], -1), np.concatenate([kf, vf], -1), vf, [Sk] * B,
                                   scale, True, (200, 0))
    check_vs_brute(out, lse, ro, rl, dt)
    # and the qv term matters: without it the output moves well past the tolerance
    o0, _ = orc.attention(q, k, v, dtype=dt, scale=scale, causal=True, window=(200, 0), nthreads=NT)
    assert np.abs(f(o0, dt) - ro).max() > 10 * TOL[dt]
    # soft capping applies to the whole score q.k + qv.v
    out, lse = orc.attention(q, k, v, dtype=dt, scale=scale, causal=True, qv=qv, softcap=3.0, nthreads=NT)
    ro, rl = brute.attention_batch(np.concatenate([qf, qvf], -1), np.concatenate([kf, vf], -1), vf, [Sk] * B,
                                   scale, True, softcap=3.0)
    check_vs_brute(out, lse, ro, rl, dt)


def test_qv_varlen_rows_follow_cu_seqlens_q():
    rng = np.random.default_rng(73)
    dt = orc.FP16
    D, H, Hk = 64, 4, 2
    cu = np.array([0, 3, 3, 7], dtype=np.int32)
    q, qv = rbits(rng, (7, H, D), dt), rbits(rng, (7, H, D), dt)
    k, v = rbits(rng, (3, 90, Hk, D), dt), rbits(rng, (3, 90, Hk, D), dt)
    seqlens = np.array([90, 50, 20], dtype=np.int32)
    o, l = orc.attention(q, k, v, dtype=dt, scale=0.1, causal=True, cu_seqlens_q=cu, seqlens_k=seqlens, qv=qv)
    for b in (0, 2):
        ob, lb = orc.attention(q[None, cu[b]:cu[b + 1]], k[b:b + 1, :seqlens[b]], v[b:b + 1, :seqlens[b]],
                               dtype=dt, scale=0.1, causal=True, qv=qv[None, cu[b]:cu[b + 1]])
        assert np.array_equal(o[cu[b]:cu[b + 1]], ob[0])
        assert np.array_equal(l[:, cu[b]:cu[b + 1]], lb[0])
