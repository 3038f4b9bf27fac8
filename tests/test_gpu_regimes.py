"""GPU parity in the regimes the benchmarks run, and the exactness claims:

* BASELINE config 4 at its full size (B4, 2048 new tokens appended at 6144
  into an 8192-slot cache, H32/8, D128, bf16, NeoX rotary, causal): the
  unsplit prefill path (about 100 key tiles per work item) with the
  automatic plan, against the CPU oracle on four (batch, kv head) slices,
  and the whole cache bit for bit;
* the paged gather is bit-exact: a paged cache (permuted block table) and a
  contiguous cache with equal contents give identical out / LSE bits and
  identical cache contents after the append;
* the append when new tokens outnumber the query rows under a left window or
  an attention chunk, and with ragged q holding an empty sequence: every new
  token reaches the cache;
* a full cache: the tokens that do not fit are dropped by both append paths
  (inside the decode kernel and the separate append kernel);
* batches above 2048 sequences (run as chunks of launches).

Reference semantics: README.md:100-109 (append, rotary) and
tests/test_flash_attn_npu_v3.py:276-521, :444-460 (kvcache test, paged gather
golden) of the reference."""
import os

import numpy as np
import pytest
import torch

from oracle import fa_oracle as orc
from tests._util import assert_close_lse, assert_close_out, bits, odt, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
NT = min(16, os.cpu_count() or 1)


def _rope(n, rd, dtype, base=10000.0):
    inv = 1.0 / (base ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd))
    ang = torch.arange(n, dtype=torch.float32)[:, None] * inv[None, :]
    return torch.cos(ang).to(dtype), torch.sin(ang).to(dtype)


# ---- BASELINE config 4 at full size --------------------------------------------------------------
def test_c4_full_size_unsplit_prefill():
    import flash_attn_npu_v2
    num_splits = 0
    print("case c4 full size (automatic plan: unsplit)", flush=True)
    B, S_new, L0, cap, H, Hk, D = 4, 2048, 6144, 8192, 32, 8, 128
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(404)
    q = randn((B, S_new, H, D), dtype, g, "cpu")
    kc = randn((B, cap, Hk, D), dtype, g, "cpu")
    vc = randn((B, cap, Hk, D), dtype, g, "cpu")
    kn = randn((B, S_new, Hk, D), dtype, g, "cpu")
    vn = randn((B, S_new, Hk, D), dtype, g, "cpu")
    cos, sin = _rope(cap, D, dtype)
    seqlens = np.full(B, L0, np.int32)

    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    out, lse = flash_attn_npu_v2.flash_attn_with_kvcache(
        q.to(DEV), kc_d, vc_d, k=kn.to(DEV), v=vn.to(DEV), rotary_cos=cos.to(DEV), rotary_sin=sin.to(DEV),
        cache_seqlens=torch.from_numpy(seqlens).to(DEV), causal=True, rotary_interleaved=False,
        num_splits=num_splits, return_softmax_lse=True)
    torch.cuda.synchronize()

    # the whole cache after the append, bit for bit
    rk, rv = orc.kv_append(bits(kc), bits(vc), bits(kn), bits(vn), seqlens, dtype=odt(dtype), cos=bits(cos),
                           sin=bits(sin), interleaved=False)
    assert np.array_equal(bits(kc_d), rk), "k_cache after the append is not bit-exact"
    assert np.array_equal(bits(vc_d), rv), "v_cache after the append is not bit-exact"

    # out / LSE on four (batch, kv head) slices of the 32, spread over the
    # batches and kv heads (each slice holds all 32 row tiles of its pair,
    # from the lightest, 6145 keys, to the heaviest, 8192)
    g_sz = H // Hk
    for b, hk in ((0, 0), (1, 3), (2, 4), (3, 7)):
        hs = slice(hk * g_sz, (hk + 1) * g_sz)
        ro, rl, _, _ = orc.kvcache_forward(
            bits(q[b:b + 1, :, hs]), bits(kc[b:b + 1, :, hk:hk + 1]), bits(vc[b:b + 1, :, hk:hk + 1]),
            dtype=odt(dtype), cache_seqlens=seqlens[b:b + 1], k=bits(kn[b:b + 1, :, hk:hk + 1]),
            v=bits(vn[b:b + 1, :, hk:hk + 1]), rotary_cos=bits(cos), rotary_sin=bits(sin),
            rotary_interleaved=False, causal=True, nthreads=NT)
        mx = assert_close_out(out[b:b + 1, :, hs], ro, dtype)
        rel = assert_close_lse(lse[b:b + 1, hs], rl)
        print(f"  slice b={b} hk={hk}: out max-abs {mx:.2e}, lse rel {rel:.2e}", flush=True)


# ---- paged gather == contiguous, bit for bit -----------------------------------------------------
def _paged_vs_contiguous(B, Sq, H, Hk, D, L, s_new, page, *, dtype=torch.bfloat16, rotary=None, window=(-1, -1),
                         alibi=False, batch_idx=False, seed=0):
    import flash_attn_npu_v2
    print(f"case paged==contiguous B{B} Sq{Sq} H{H}/{Hk} D{D} page{page} new{s_new} rot={rotary} "
          f"win={window} alibi={alibi} bidx={batch_idx}", flush=True)
    g = torch.Generator().manual_seed(seed)
    L = np.asarray(L, np.int32)
    rows = B + 2 if batch_idx else B
    bidx = torch.randperm(rows, generator=g)[:B].to(torch.int32) if batch_idx else None
    row_len = np.zeros(rows, np.int64)
    for b in range(B):
        row_len[int(bidx[b]) if bidx is not None else b] = int(L[b]) + s_new
    nper = (int(row_len.max()) + page - 1) // page
    cap = nper * page
    # contiguous cache rows; the paged pool holds the same pages under a permutation
    kc = randn((rows, cap, Hk, D), dtype, g, "cpu")
    vc = randn((rows, cap, Hk, D), dtype, g, "cpu")
    nblocks = rows * nper + 3
    perm = torch.randperm(nblocks, generator=g)[:rows * nper].to(torch.int32)
    bt = perm.view(rows, nper)
    kp = randn((nblocks, page, Hk, D), dtype, g, "cpu")  # pages no row uses keep random bits
    vp = randn((nblocks, page, Hk, D), dtype, g, "cpu")
    kp[bt.reshape(-1).long()] = kc.view(rows * nper, page, Hk, D)
    vp[bt.reshape(-1).long()] = vc.view(rows * nper, page, Hk, D)
    q = randn((B, Sq, H, D), dtype, g, "cpu")
    kn = randn((B, s_new, Hk, D), dtype, g, "cpu") if s_new else None
    vn = randn((B, s_new, Hk, D), dtype, g, "cpu") if s_new else None
    cos = sin = None
    if rotary:
        cos, sin = _rope(cap + Sq + 8, D, dtype)
    slopes = torch.tensor([2.0 ** (-8.0 * (h + 1) / H) for h in range(H)], dtype=torch.float32) if alibi else None
    d = lambda t: None if t is None else t.to(DEV)
    res = []
    for paged in (False, True):
        kcache, vcache = (kp.to(DEV), vp.to(DEV)) if paged else (kc.to(DEV), vc.to(DEV))
        out, lse = flash_attn_npu_v2.flash_attn_with_kvcache(
            d(q), kcache, vcache, k=d(kn), v=d(vn), rotary_cos=d(cos), rotary_sin=d(sin),
            cache_seqlens=torch.from_numpy(L).to(DEV), cache_batch_idx=d(bidx), block_table=d(bt) if paged else None,
            causal=True, window_size=window, rotary_interleaved=rotary == "interleaved", alibi_slopes=d(slopes),
            return_softmax_lse=True)
        torch.cuda.synchronize()
        if paged:  # gather the pool back into rows
            kcache = kcache[bt.to(DEV).reshape(-1).long()].view(rows, cap, Hk, D)
            vcache = vcache[bt.to(DEV).reshape(-1).long()].view(rows, cap, Hk, D)
        res.append((bits(out), lse.cpu().numpy().view(np.uint32), bits(kcache), bits(vcache)))
    (o0, l0, k0, v0), (o1, l1, k1, v1) = res
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1), "caches differ after the append"
    assert np.array_equal(o0, o1), f"out differs in {(o0 != o1).sum()} elements"
    assert np.array_equal(l0, l1), f"lse differs in {(l0 != l1).sum()} elements"


@pytest.mark.parametrize("page", [256, 64])
def test_paged_bitwise_decode(page):
    rng = np.random.default_rng(500 + page)
    L = np.round(np.exp(rng.uniform(np.log(512), np.log(9000), size=12))).astype(np.int32)
    _paged_vs_contiguous(12, 1, 64, 8, 128, L, 1, page, seed=500 + page)


@pytest.mark.parametrize("page", [256, 64])
def test_paged_bitwise_chunked_prefill_rotary(page):
    _paged_vs_contiguous(2, 300, 32, 8, 128, [1000, 2500], 300, page, rotary="neox", seed=510 + page)


def test_paged_bitwise_verify_window_alibi_batch_idx():
    rng = np.random.default_rng(520)
    _paged_vs_contiguous(6, 4, 32, 8, 128, rng.integers(3000, 9000, 6), 0, 256, window=(2048, 0), alibi=True,
                         batch_idx=True, seed=520)


def test_paged_bitwise_headdim64_decode():
    rng = np.random.default_rng(530)
    _paged_vs_contiguous(8, 1, 32, 8, 64, rng.integers(100, 5000, 8), 1, 64, dtype=torch.float16, seed=530)


# ---- appends the decode kernel cannot fuse --------------------------------------------------------
def test_append_more_new_tokens_than_rows_left_window():
    from tests.test_gpu_v3kv import run_v3
    # one query row, two new tokens, window (0, 0): the first new token lies
    # left of every visited key tile
    run_v3(H=8, Hk=2, q_lens=[1] * 3, new_lens=[2] * 3, seqlens=[31, 5, 40], capacity=64, window=(0, 0), seed=540)


def test_append_more_new_tokens_than_rows_chunk():
    from tests.test_gpu_v3kv import run_v3
    run_v3(H=8, Hk=2, q_lens=[1] * 3, new_lens=[5] * 3, seqlens=[60, 3, 200], capacity=256, chunk=32, seed=541)


def test_append_ragged_q_with_empty_sequence():
    from tests.test_gpu_v3kv import run_v3
    # sequence 1 has no query rows (no key tiles) but two new tokens
    run_v3(H=8, Hk=2, q_lens=[2, 0, 1], new_lens=[2] * 3, seqlens=[100, 37, 500], capacity=640, ragged_q=True,
           seed=542)


@pytest.mark.parametrize("window", [(-1, -1), (8, 0)])
def test_append_dense_empty_q(window):
    """A (B, 0, H, D) q with new k / v: no attention runs, yet every new token
    reaches the cache, with and without a left window."""
    import flash_attn_npu_v2
    print(f"case empty q with append, window {window}", flush=True)
    B, H, Hk, D, cap, s_new = 3, 8, 2, 128, 64, 2
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(543)
    L = np.array([5, 30, 61], np.int32)
    q = torch.empty((B, 0, H, D), dtype=dtype)
    kc = randn((B, cap, Hk, D), dtype, g, "cpu")
    vc = randn((B, cap, Hk, D), dtype, g, "cpu")
    kn = randn((B, s_new, Hk, D), dtype, g, "cpu")
    vn = randn((B, s_new, Hk, D), dtype, g, "cpu")
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    out, lse = flash_attn_npu_v2.flash_attn_with_kvcache(
        q.to(DEV), kc_d, vc_d, k=kn.to(DEV), v=vn.to(DEV), cache_seqlens=torch.from_numpy(L).to(DEV), causal=True,
        window_size=window, return_softmax_lse=True)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (B, 0, H, D) and tuple(lse.shape) == (B, H, 0)
    ek, ev = bits(kc).copy(), bits(vc).copy()
    for b in range(B):
        ek[b, L[b]:L[b] + s_new] = bits(kn)[b]
        ev[b, L[b]:L[b] + s_new] = bits(vn)[b]
    assert np.array_equal(bits(kc_d), ek) and np.array_equal(bits(vc_d), ev), "new tokens missing from the cache"


# ---- a full cache: both append paths drop what does not fit ---------------------------------------
def test_full_cache_append_paths_agree():
    import flash_attn_npu_v2
    print("case full cache: fused vs separate append", flush=True)
    B, Sq, H, Hk, D, cap, s_new = 3, 3, 8, 2, 128, 96, 3
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(550)
    L = np.array([cap - 1, cap - 2, 10], np.int32)
    q = randn((B, Sq, H, D), dtype, g, "cpu")
    kc = randn((B, cap, Hk, D), dtype, g, "cpu")
    vc = randn((B, cap, Hk, D), dtype, g, "cpu")
    kn = randn((B, s_new, Hk, D), dtype, g, "cpu")
    vn = randn((B, s_new, Hk, D), dtype, g, "cpu")
    # rotary with cos = 1, sin = 0 is the identity, but sends the call through
    # the separate append kernel
    ones = torch.ones((cap + 8, D // 2), dtype=dtype)
    zeros = torch.zeros((cap + 8, D // 2), dtype=dtype)
    res = []
    for rot in (False, True):
        kc_d, vc_d = kc.to(DEV), vc.to(DEV)
        out, lse = flash_attn_npu_v2.flash_attn_with_kvcache(
            q.to(DEV), kc_d, vc_d, k=kn.to(DEV), v=vn.to(DEV), cache_seqlens=torch.from_numpy(L).to(DEV),
            rotary_cos=ones.to(DEV) if rot else None, rotary_sin=zeros.to(DEV) if rot else None, causal=True,
            return_softmax_lse=True)
        torch.cuda.synchronize()
        res.append((bits(out), lse.cpu().numpy(), bits(kc_d), bits(vc_d)))
    # expected: the tokens that fit are appended, attention covers min(L + s_new, cap) keys
    ek, ev = bits(kc).copy(), bits(vc).copy()
    for b in range(B):
        n = min(s_new, cap - int(L[b]))
        ek[b, L[b]:L[b] + n] = bits(kn)[b, :n]
        ev[b, L[b]:L[b] + n] = bits(vn)[b, :n]
    ro, rl = orc.attention(bits(q), ek, ev, dtype=odt(dtype), scale=D ** -0.5, causal=True,
                           seqlens_k=np.minimum(L + s_new, cap).astype(np.int32), nthreads=NT)
    for o, l, k, v in res:
        assert np.array_equal(k, ek) and np.array_equal(v, ev), "cache differs from the drop-what-does-not-fit rule"
        assert_close_out(torch.from_numpy(o.view(np.int16)).view(dtype), ro, dtype)
        assert_close_lse(torch.from_numpy(l), rl)
    assert np.array_equal(res[0][0], res[1][0]) and np.array_equal(res[0][1], res[1][1]), "the two paths differ"


# ---- more than 2048 sequences in one call ---------------------------------------------------------
def test_varlen_prefill_3000_sequences():
    import flash_attn_npu_v2
    print("case varlen B=3000", flush=True)
    g = torch.Generator().manual_seed(560)
    rng = np.random.default_rng(560)
    dtype = torch.bfloat16
    B, H, Hk, D = 3000, 4, 1, 64
    lq = rng.integers(1, 9, B)
    lk = lq + rng.integers(0, 6, B)
    cq = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    ck = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
    q = randn((int(cq[-1]), H, D), dtype, g, "cpu")
    k = randn((int(ck[-1]), Hk, D), dtype, g, "cpu")
    v = randn((int(ck[-1]), Hk, D), dtype, g, "cpu")
    ro, rl = orc.attention(bits(q), bits(k), bits(v), dtype=odt(dtype), scale=D ** -0.5, causal=True,
                           cu_seqlens_q=cq, cu_seqlens_k=ck, max_seqlen_q=int(lq.max()), nthreads=NT)
    out, lse, _ = flash_attn_npu_v2.flash_attn_varlen_func(
        q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(cq).to(DEV), torch.from_numpy(ck).to(DEV), int(lq.max()),
        int(lk.max()), causal=True, return_attn_probs=True)
    torch.cuda.synchronize()
    assert_close_out(out, ro, dtype)
    assert_close_lse(lse, rl)


def test_decode_2500_sequences_append():
    from tests.test_gpu_parity import run_kvcache
    print("case decode B=2500", flush=True)
    rng = np.random.default_rng(561)
    run_kvcache(2500, 1, 8, 2, 128, torch.bfloat16, 160, rng.integers(0, 150, 2500), s_new=1, causal=True,
                seed=561)


def test_backward_dense_2100_sequences():
    import flash_attn_npu_v2
    from oracle import fa_bwd_oracle as bo
    print("case backward B=2100", flush=True)
    g = torch.Generator().manual_seed(562)
    B, S, H, Hk, D = 2100, 8, 2, 1, 64
    mk = lambda *s: (2 * (torch.rand(s, generator=g) - 0.5)).to(torch.bfloat16)
    q, k, v, do = mk(B, S, H, D), mk(B, S, Hk, D), mk(B, S, Hk, D), mk(B, S, H, D)
    qd, kd, vd = (x.to(DEV).requires_grad_(True) for x in (q, k, v))
    out, lse, _ = flash_attn_npu_v2.flash_attn_func(qd, kd, vd, causal=True, return_attn_probs=True)
    grads = torch.autograd.grad(out, (qd, kd, vd), do.to(DEV))
    torch.cuda.synchronize()
    refs = bo.attention_bwd(q.float().numpy(), k.float().numpy(), v.float().numpy(), do.float().numpy(),
                            lse.detach().cpu().numpy(), scale=D ** -0.5, causal=True)
    for name, got, ref in zip(("dq", "dk", "dv"), grads, refs):
        dif = np.abs(got.float().cpu().numpy() - ref)
        assert (dif <= 1e-2 + 1e-2 * np.abs(ref)).all(), f"{name}: max err {dif.max():.3e}"
