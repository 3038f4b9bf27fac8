"""GPU parity: the HIP path (through the C ABI, via the public APIs) against
the CPU oracle on identical seeded inputs. Tolerances are the north-star ones:
out max-abs <= 2e-3 (fp16) / 1e-2 (bf16) against the golden, softmax LSE
within 1e-4 relative, cache append and paged gather bit-exact."""
import os

import numpy as np
import pytest
import torch

from oracle import fa_oracle as orc
from tests._util import assert_close_lse, assert_close_out, bits, odt, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
NT = min(16, os.cpu_count() or 1)


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def run_kvcache(B, Sq, H, Hk, D, dtype, capacity, seqlens, s_new=0, page=0, rotary=None, causal=True,
                window=(-1, -1), alibi=False, batch_idx=False, num_splits=0, softcap=0.0, seed=0, api="v2"):
    import flash_attn_npu_v2
    import flash_attn_npu_v3
    g = _gen(seed)
    seqlens = np.asarray(seqlens, dtype=np.int32)
    q = randn((B, Sq, H, D), dtype, g, "cpu")
    bc = B
    bidx = None
    if batch_idx:
        bc = B + 2
        bidx = torch.randperm(bc, generator=g)[:B].to(torch.int32)
    if page:
        need = [(int(L) + s_new + page - 1) // page for L in seqlens]
        rows = bc
        row_need = [0] * rows
        for b in range(B):
            r = int(bidx[b]) if bidx is not None else b
            row_need[r] = need[b]
        max_blocks = max(max(row_need), 1)
        nblocks = sum(row_need) + max(2, sum(row_need) // 10)
        perm = torch.randperm(nblocks, generator=g).to(torch.int32)
        bt = torch.zeros((rows, max_blocks), dtype=torch.int32)
        o = 0
        for r in range(rows):
            bt[r, :row_need[r]] = perm[o:o + row_need[r]]
            o += row_need[r]
        kc = randn((nblocks, page, Hk, D), dtype, g, "cpu")
        vc = randn((nblocks, page, Hk, D), dtype, g, "cpu")
    else:
        bt = None
        kc = randn((bc, capacity, Hk, D), dtype, g, "cpu")
        vc = randn((bc, capacity, Hk, D), dtype, g, "cpu")
    kn = vn = None
    if s_new:
        kn = randn((B, s_new, Hk, D), dtype, g, "cpu")
        vn = randn((B, s_new, Hk, D), dtype, g, "cpu")
    cos = sin = None
    if rotary:
        rd = D if rotary != "partial" else D // 2
        ro_len = (max(int(L) for L in seqlens) + s_new + Sq + 8)
        inv = 1.0 / (10000 ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd))
        ang = torch.arange(ro_len, dtype=torch.float32)[:, None] * inv[None, :]
        cos, sin = torch.cos(ang).to(dtype), torch.sin(ang).to(dtype)
    slopes = None
    if alibi:
        slopes = torch.tensor([2.0 ** (-8.0 * (h + 1) / H) for h in range(H)], dtype=torch.float32)
    interleaved = rotary == "interleaved"

    # oracle on host bits
    ref_out, ref_lse, ref_kc, ref_vc = orc.kvcache_forward(
        bits(q).reshape(q.shape), bits(kc).reshape(kc.shape), bits(vc).reshape(vc.shape), dtype=odt(dtype),
        cache_seqlens=seqlens, k=None if kn is None else bits(kn).reshape(kn.shape),
        v=None if vn is None else bits(vn).reshape(vn.shape),
        rotary_cos=None if cos is None else bits(cos).reshape(cos.shape),
        rotary_sin=None if sin is None else bits(sin).reshape(sin.shape), rotary_interleaved=interleaved,
        cache_batch_idx=None if bidx is None else bidx.numpy(), block_table=None if bt is None else bt.numpy(),
        causal=causal, window=window, softcap=softcap, alibi=None if slopes is None else slopes.numpy(),
        nthreads=NT)

    d = lambda t: None if t is None else t.to(DEV)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    sl_d = torch.from_numpy(seqlens).to(DEV)
    if api == "v2":
        out, lse = flash_attn_npu_v2.flash_attn_with_kvcache(
            d(q), kc_d, vc_d, k=d(kn), v=d(vn), rotary_cos=d(cos), rotary_sin=d(sin), cache_seqlens=sl_d,
            cache_batch_idx=d(bidx), block_table=d(bt), causal=causal, window_size=window, softcap=softcap,
            rotary_interleaved=interleaved, alibi_slopes=d(slopes), num_splits=num_splits, return_softmax_lse=True)
    else:
        out, lse, *_ = flash_attn_npu_v3.flash_attn_with_kvcache(
            d(q), kc_d, vc_d, k=d(kn), v=d(vn), rotary_cos=d(cos), rotary_sin=d(sin), cache_seqlens=sl_d,
            cache_batch_idx=d(bidx), page_table=d(bt), causal=causal, window_size=window, softcap=softcap,
            rotary_interleaved=interleaved, num_splits=num_splits, return_softmax_lse=True)
    torch.cuda.synchronize()
    if s_new:
        assert np.array_equal(bits(kc_d).reshape(kc.shape), ref_kc), "k_cache append is not bit-exact"
        assert np.array_equal(bits(vc_d).reshape(vc.shape), ref_vc), "v_cache append is not bit-exact"
    mx = assert_close_out(out, ref_out, dtype)
    rl = assert_close_lse(lse, ref_lse)
    return mx, rl


def run_dense(B, Sq, Sk, H, Hk, D, dtype, causal=True, window=(-1, -1), softcap=0.0, alibi=False, seed=0):
    import flash_attn_npu_v2
    g = _gen(seed)
    q = randn((B, Sq, H, D), dtype, g, "cpu")
    k = randn((B, Sk, Hk, D), dtype, g, "cpu")
    v = randn((B, Sk, Hk, D), dtype, g, "cpu")
    slopes = torch.tensor([2.0 ** (-8.0 * (h + 1) / H) for h in range(H)], dtype=torch.float32) if alibi else None
    scale = D ** -0.5
    ref_out, ref_lse = orc.attention(bits(q).reshape(q.shape), bits(k).reshape(k.shape), bits(v).reshape(v.shape),
                                     dtype=odt(dtype), scale=scale, softcap=softcap, causal=causal, window=window,
                                     alibi=None if slopes is None else slopes.numpy(), nthreads=NT)
    out, lse, _ = flash_attn_npu_v2.flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal,
                                                    window_size=window, softcap=softcap,
                                                    alibi_slopes=None if slopes is None else slopes.to(DEV),
                                                    return_attn_probs=True)
    torch.cuda.synchronize()
    assert_close_out(out, ref_out, dtype)
    assert_close_lse(lse, ref_lse)


# ---- BASELINE config 1 (the parity anchor) at full size -------------------------------------
def test_c1_dense_causal_fp16():
    print("case c1: B2 S512 H16 D128 fp16 causal", flush=True)
    run_dense(2, 512, 512, 16, 16, 128, torch.float16, causal=True, seed=1)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
def test_dense_gqa(dtype, causal):
    print(f"case dense gqa {dtype} causal={causal}", flush=True)
    run_dense(2, 200, 333, 8, 2, 128, dtype, causal=causal, seed=2)


def test_dense_sq_gt_sk_empty_rows():
    # seqlen_q > seqlen_k with causal: the first rows see no key -> out 0, lse +inf
    print("case dense sq>sk", flush=True)
    run_dense(1, 70, 40, 4, 4, 128, torch.bfloat16, causal=True, seed=3)


def test_dense_window_softcap_alibi():
    print("case dense window+softcap+alibi", flush=True)
    run_dense(2, 160, 300, 8, 4, 128, torch.bfloat16, causal=False, window=(50, 20), softcap=30.0, alibi=True, seed=4)


# ---- decode (3, 5 shapes, reduced lengths) -------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_contiguous_append(dtype):
    print(f"case decode contiguous append {dtype}", flush=True)
    g = np.random.default_rng(5)
    seqlens = g.integers(1, 2000, size=8)
    run_kvcache(8, 1, 32, 8, 128, dtype, 2048, seqlens, s_new=1, causal=True, seed=5)


@pytest.mark.parametrize("num_splits", [0, 1, 3])
def test_decode_paged_split(num_splits):
    print(f"case decode paged num_splits={num_splits}", flush=True)
    g = np.random.default_rng(6)
    seqlens = np.round(np.exp(g.uniform(np.log(16), np.log(3000), size=6))).astype(np.int32)
    run_kvcache(6, 1, 64, 8, 128, torch.bfloat16, 0, seqlens, s_new=1, page=256, causal=True,
                num_splits=num_splits, seed=6)


def test_specverify_paged_window_alibi_batchidx():
    print("case spec-verify paged window alibi cache_batch_idx", flush=True)
    g = np.random.default_rng(7)
    seqlens = g.integers(1500, 4000, size=4)
    run_kvcache(4, 4, 32, 8, 128, torch.bfloat16, 0, seqlens, s_new=0, page=256, causal=True,
                window=(600, 0), alibi=True, batch_idx=True, seed=7)


# ---- chunked prefill with rotary (BASELINE config 4 shape, reduced) ---------------------------
@pytest.mark.parametrize("rotary", ["neox", "interleaved"])
def test_chunked_prefill_rotary(rotary):
    print(f"case chunked prefill rotary={rotary}", flush=True)
    run_kvcache(2, 96, 16, 4, 128, torch.bfloat16, 512, [300, 111], s_new=96, rotary=rotary, causal=True, seed=8)


def test_v3_kvcache_paged():
    print("case v3 kvcache paged", flush=True)
    run_kvcache(3, 2, 16, 4, 128, torch.float16, 0, [100, 700, 1300], s_new=2, page=64, causal=True, seed=9,
                api="v3")
