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


def test_decode_paged_split():
    # a forced num_splits cuts every sequence's keys into that many chunks (the
    # split prefill path) instead of the decode kernel's stream-K split
    print("case decode paged num_splits=3", flush=True)
    g = np.random.default_rng(6)
    seqlens = np.round(np.exp(g.uniform(np.log(16), np.log(3000), size=6))).astype(np.int32)
    run_kvcache(6, 1, 64, 8, 128, torch.bfloat16, 0, seqlens, s_new=1, page=256, causal=True, num_splits=3, seed=6)


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


# ---- head dims below 128 (dims above D are zero inside the kernels, never written) -----------
@pytest.mark.parametrize("D", [64, 80, 96])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_headdim_dense(D, dtype):
    print(f"case headdim dense D={D} {dtype}", flush=True)
    run_dense(2, 150, 260, 8, 2, D, dtype, causal=True, seed=40 + D)


@pytest.mark.parametrize("D", [64, 96])
def test_headdim_decode_paged_append(D):
    print(f"case headdim decode paged D={D}", flush=True)
    run_kvcache(5, 1, 32, 8, D, torch.bfloat16, 0, [700, 33, 4000, 1, 2500], s_new=1, page=64, causal=True,
                seed=50 + D)


def test_headdim_decode_contiguous_fused_append_large():
    print("case headdim decode contiguous D=64 large", flush=True)
    rng = np.random.default_rng(52)
    run_kvcache(16, 1, 32, 8, 64, torch.float16, 8192, rng.integers(1024, 8191, size=16), s_new=1, causal=True,
                seed=52)


@pytest.mark.parametrize("rotary", ["neox", "interleaved"])
def test_headdim_chunked_prefill_rotary(rotary):
    print(f"case headdim 64 chunked prefill rotary {rotary}", flush=True)
    run_kvcache(2, 80, 16, 4, 64, torch.bfloat16, 400, [200, 57], s_new=80, rotary=rotary, causal=True, seed=53)


# ---- head dims up to 64: the 64 prefill kernel (64 rows per wave, 128-byte LDS rows) ---------
@pytest.mark.parametrize("D", [32, 48, 64])
def test_headdim64_dense_noncausal(D):
    print(f"case headdim64 dense non-causal D={D}", flush=True)
    run_dense(2, 300, 170, 8, 4, D, torch.bfloat16, causal=False, seed=70 + D)


def test_headdim64_window_softcap_alibi():
    print("case headdim64 window softcap alibi", flush=True)
    run_dense(2, 257, 600, 8, 2, 64, torch.float16, causal=True, window=(100, 0), softcap=20.0, alibi=True, seed=74)


def test_headdim64_split_few_rows():
    print("case headdim64 split over the keys", flush=True)
    run_dense(1, 40, 5000, 4, 1, 64, torch.bfloat16, causal=True, seed=75)


def test_headdim64_paged_chunked_prefill_rotary():
    print("case headdim64 paged chunked prefill rotary", flush=True)
    run_kvcache(3, 70, 16, 4, 64, torch.bfloat16, 0, [300, 0, 129], s_new=70, page=32, rotary="neox", causal=True,
                seed=76)


# ---- decode at head dims up to 64: 64-key tiles, 128-byte LDS rows ----------------------------
@pytest.mark.parametrize("D,page", [(64, 32), (32, 128), (48, 0), (64, 0)])
def test_headdim64_decode_layouts(D, page):
    print(f"case headdim64 decode D={D} page={page}", flush=True)
    rng = np.random.default_rng(80 + D + page)
    run_kvcache(6, 1, 32, 8, D, torch.bfloat16, 0 if page else 3000, rng.integers(1, 2900, size=6), s_new=1,
                page=page, causal=True, seed=80 + D + page)


def test_headdim64_decode_verify_window_alibi_softcap():
    print("case headdim64 decode verify window alibi softcap", flush=True)
    rng = np.random.default_rng(84)
    run_kvcache(4, 4, 16, 4, 64, torch.float16, 0, rng.integers(700, 5000, size=4), s_new=4, page=64, causal=True,
                window=(500, 0), alibi=True, softcap=30.0, batch_idx=True, seed=84)


# ---- head dims above 128: the 256 prefill kernel (decode shapes run on it too) --------------
@pytest.mark.parametrize("D", [136, 192, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_headdim_large_dense(D, dtype):
    print(f"case headdim dense D={D} {dtype}", flush=True)
    run_dense(2, 150, 260, 8, 2, D, dtype, causal=True, seed=60 + D)


def test_headdim_256_dense_window_softcap_alibi():
    print("case headdim 256 dense window softcap alibi", flush=True)
    run_dense(2, 200, 333, 8, 4, 256, torch.bfloat16, causal=False, window=(90, 30), softcap=30.0, alibi=True,
              seed=61)


@pytest.mark.parametrize("D", [192, 256])
def test_headdim_large_decode_paged_append(D):
    # reference v3 decode cases at D=256 (tests/test_flash_attn_npu_v3.py:193,207)
    print(f"case headdim {D} decode paged append", flush=True)
    run_kvcache(5, 1, 32, 8, D, torch.bfloat16, 0, [700, 33, 4000, 1, 2500], s_new=1, page=64, causal=True,
                seed=62 + D)


def test_headdim_256_decode_contiguous_long():
    print("case headdim 256 decode contiguous long (split)", flush=True)
    run_kvcache(2, 1, 64, 8, 256, torch.bfloat16, 4096, [4000, 2048], s_new=1, causal=True, seed=63)


def test_headdim_256_spec_verify_window_alibi_batchidx():
    print("case headdim 256 verify paged window alibi batch_idx", flush=True)
    run_kvcache(4, 13, 32, 8, 256, torch.bfloat16, 0, [1500, 2600, 900, 3000], s_new=0, page=128, causal=True,
                window=(600, 0), alibi=True, batch_idx=True, seed=64)


@pytest.mark.parametrize("rotary", ["neox", "interleaved", "partial"])
def test_headdim_256_chunked_prefill_rotary(rotary):
    print(f"case headdim 256 chunked prefill rotary {rotary}", flush=True)
    run_kvcache(2, 70, 16, 4, 256, torch.bfloat16, 400, [200, 57], s_new=70, rotary=rotary, causal=True, seed=65)


def test_headdim_256_varlen():
    import flash_attn_npu_v3
    print("case headdim 256 varlen", flush=True)
    g = _gen(66)
    dtype = torch.bfloat16
    H, Hk, D = 8, 2, 256
    lq = [37, 1, 300, 64]
    lk = [37, 90, 300, 700]
    cq = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    ck = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
    q = randn((cq[-1], H, D), dtype, g, "cpu")
    k = randn((ck[-1], Hk, D), dtype, g, "cpu")
    v = randn((ck[-1], Hk, D), dtype, g, "cpu")
    ref_out, ref_lse = orc.attention(bits(q).reshape(q.shape), bits(k).reshape(k.shape), bits(v).reshape(v.shape),
                                     dtype=odt(dtype), scale=D ** -0.5, causal=True, cu_seqlens_q=cq,
                                     cu_seqlens_k=ck, max_seqlen_q=max(lq), nthreads=NT)
    out, lse = flash_attn_npu_v3.flash_attn_varlen_func(
        q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(cq).to(DEV), torch.from_numpy(ck).to(DEV), max(lq),
        max(lk), causal=True, return_attn_probs=True)
    torch.cuda.synchronize()
    assert_close_out(out, ref_out, dtype)
    assert_close_lse(lse, ref_lse)


def test_headdim_padded_to_multiple_of_8():
    # the v2 API pads the head dim to a multiple of 8 and slices the output (interface_arch22.py:1102-1176)
    import flash_attn_npu_v2
    print("case headdim 36 padded", flush=True)
    g = _gen(54)
    q = randn((2, 40, 4, 36), torch.float16, g, "cpu")
    k = randn((2, 70, 2, 36), torch.float16, g, "cpu")
    v = randn((2, 70, 2, 36), torch.float16, g, "cpu")
    ref_out, ref_lse = orc.attention(bits(q).reshape(q.shape), bits(k).reshape(k.shape), bits(v).reshape(v.shape),
                                     dtype=orc.FP16, scale=36 ** -0.5, causal=True, nthreads=NT)
    out, lse, _ = flash_attn_npu_v2.flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), causal=True,
                                                    return_attn_probs=True)
    torch.cuda.synchronize()
    assert out.shape == q.shape
    assert_close_out(out, ref_out, torch.float16)
    assert_close_lse(lse, ref_lse)


# ---- split-KV merge: repeated calls reuse the workspace ------------------------------------------
def test_split_repeated_calls():
    print("case repeated split calls", flush=True)
    for rep in range(3):
        run_kvcache(5, 1, 32, 8, 128, torch.bfloat16, 4096, [4000, 100, 2500, 3000, 1], s_new=1, causal=True,
                    num_splits=0, seed=20)


# ---- decode at scale: thousands of 32-key tiles, segments cut by many wave workers ------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_large_contiguous(dtype):
    print(f"case large decode contiguous {dtype}", flush=True)
    rng = np.random.default_rng(31)
    seqlens = rng.integers(1024, 8191, size=16)
    for rep in range(2):
        run_kvcache(16, 1, 32, 8, 128, dtype, 8192, seqlens, s_new=1, causal=True, seed=31 + rep)


def test_decode_large_paged_uneven():
    print("case large decode paged uneven", flush=True)
    rng = np.random.default_rng(32)
    seqlens = np.round(np.exp(rng.uniform(np.log(512), np.log(32768), size=12))).astype(np.int64)
    run_kvcache(12, 1, 64, 8, 128, torch.bfloat16, 0, seqlens, s_new=1, page=256, causal=True, seed=32)


def test_decode_many_segments_cost_split():
    # 64 x 8 = 512 (sequence, kv head) segments over 1024 waves, in the
    # kernel's groups of 4 kv heads 128 group segments over 256 wave groups,
    # with at least 16 tiles each: the regime of BASELINE config 3, where the
    # decode split counts every segment as one extra tile and a worker's first
    # partial and latest whole output are held until it ends
    print("case decode many segments (split by cost)", flush=True)
    rng = np.random.default_rng(35)
    seqlens = np.round(np.exp(rng.uniform(np.log(512), np.log(8192), size=64))).astype(np.int64)
    assert 64 * 8 * int(np.mean(seqlens)) // 32 >= 16 * 1024
    run_kvcache(64, 1, 64, 8, 128, torch.bfloat16, 0, seqlens, s_new=1, page=256, causal=True, seed=35)


# ---- kv head groups: the 4 waves of a CU stream 4 adjacent kv heads of one tile range when
# nheads_k % 4 == 0, pairs of waves 2 heads when it is otherwise even, else one head each; the
# tile split and the merge of the partials run over those groups
@pytest.mark.parametrize("Hk", [1, 2, 3, 4, 6, 12, 16])
@pytest.mark.parametrize("page", [0, 64])
@pytest.mark.parametrize("Sq", [1, 4])
def test_decode_kv_head_groups(Hk, page, Sq):
    print(f"case decode kv head groups Hk={Hk} page={page} Sq={Sq}", flush=True)
    rng = np.random.default_rng(40 + Hk)
    seqlens = rng.integers(1, 6000, size=6)
    seqlens[:3] = [1, 33, 5999]
    run_kvcache(6, Sq, 2 * Hk, Hk, 128, torch.bfloat16, 0 if page else 6144, seqlens, s_new=Sq, page=page,
                causal=True, seed=40 + Hk)


@pytest.mark.parametrize("Hk,B", [(6, 96), (12, 48)])
def test_decode_kv_head_groups_cost_split(Hk, B):
    # groups of 2 (Hk 6) and 4 (Hk 12) kv heads with at least half a group
    # segment and 16 tiles per wave group on a 256-CU part: the split by cost
    print(f"case decode kv head groups cost split Hk={Hk} B={B}", flush=True)
    rng = np.random.default_rng(50 + Hk)
    seqlens = rng.integers(1000, 3000, size=B)
    run_kvcache(B, 1, 2 * Hk, Hk, 128, torch.bfloat16, 0, seqlens, s_new=1, page=64, causal=True, seed=50 + Hk)


def test_decode_one_long_sequence():
    # one (sequence, kv head) segment spans every wave worker: the merge combines ~1024 partials
    print("case decode one long sequence", flush=True)
    run_kvcache(1, 1, 8, 1, 128, torch.bfloat16, 140000, [139000], s_new=1, causal=True, seed=33)


def test_decode_large_verify_window_alibi():
    print("case large spec-verify window alibi", flush=True)
    rng = np.random.default_rng(34)
    seqlens = rng.integers(16384, 65536, size=8)
    run_kvcache(8, 4, 32, 8, 128, torch.bfloat16, 0, seqlens, s_new=0, page=256, causal=True, window=(4096, 0),
                alibi=True, batch_idx=True, seed=34)


def test_prefill_shape_split_small_batch():
    # 64 query rows x g=4 -> the 128-row prefill kernel, few tiles -> auto split
    print("case prefill-shape split", flush=True)
    run_kvcache(1, 64, 32, 8, 128, torch.bfloat16, 4096, [3900], s_new=0, causal=True, seed=21)


def test_forced_split_window_empty_splits():
    print("case forced split with window", flush=True)
    run_kvcache(3, 2, 16, 4, 128, torch.float16, 0, [3000, 5000, 700], s_new=2, page=128, causal=True,
                window=(300, 0), num_splits=7, seed=22)


def test_contiguous_cache_batch_idx_append():
    print("case contiguous cache_batch_idx", flush=True)
    run_kvcache(4, 3, 16, 4, 128, torch.bfloat16, 1024, [10, 500, 900, 0], s_new=3, causal=True, batch_idx=True,
                seed=23)


def test_noncausal_decode_rotary_same_position():
    # not causal and not local: every q row is rotated at cache_seqlens[b]
    print("case non-causal rotary", flush=True)
    run_kvcache(2, 3, 16, 4, 128, torch.bfloat16, 512, [100, 200], s_new=3, rotary="partial", causal=False, seed=24)


# ---- varlen ---------------------------------------------------------------------------------
@pytest.mark.parametrize("causal", [False, True])
def test_varlen(causal):
    import flash_attn_npu_v2
    print(f"case varlen causal={causal}", flush=True)
    g = _gen(30)
    dtype = torch.bfloat16
    H, Hk, D = 8, 2, 128
    lq = [37, 1, 300, 128]
    lk = [37, 90, 300, 1000]
    cq = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    ck = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
    q = randn((cq[-1], H, D), dtype, g, "cpu")
    k = randn((ck[-1], Hk, D), dtype, g, "cpu")
    v = randn((ck[-1], Hk, D), dtype, g, "cpu")
    ref_out, ref_lse = orc.attention(bits(q).reshape(q.shape), bits(k).reshape(k.shape), bits(v).reshape(v.shape),
                                     dtype=odt(dtype), scale=D ** -0.5, causal=causal, cu_seqlens_q=cq,
                                     cu_seqlens_k=ck, max_seqlen_q=max(lq), nthreads=NT)
    out, lse, _ = flash_attn_npu_v2.flash_attn_varlen_func(
        q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(cq).to(DEV), torch.from_numpy(ck).to(DEV), max(lq),
        max(lk), causal=causal, return_attn_probs=True)
    torch.cuda.synchronize()
    assert_close_out(out, ref_out, dtype)
    assert_close_lse(lse, ref_lse)


def test_v3_varlen_q_paged_kvcache():
    import flash_attn_npu_v3
    print("case v3 TND q against paged cache", flush=True)
    g = _gen(31)
    dtype = torch.float16
    H, Hk, D, page = 8, 2, 128, 64
    lq = [3, 1, 7]
    L = [200, 64, 1000]
    need = [(x + page - 1) // page for x in L]
    nb = sum(need) + 3
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt = torch.zeros((3, max(need)), dtype=torch.int32)
    o = 0
    for b in range(3):
        bt[b, :need[b]] = perm[o:o + need[b]]
        o += need[b]
    cq = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    q = randn((cq[-1], H, D), dtype, g, "cpu")
    kc = randn((nb, page, Hk, D), dtype, g, "cpu")
    vc = randn((nb, page, Hk, D), dtype, g, "cpu")
    ref_out, ref_lse = orc.attention(bits(q).reshape(q.shape), bits(kc).reshape(kc.shape),
                                     bits(vc).reshape(vc.shape), dtype=odt(dtype), scale=D ** -0.5, causal=True,
                                     cu_seqlens_q=cq, max_seqlen_q=max(lq), seqlens_k=np.array(L, np.int32),
                                     block_table=bt.numpy(), nthreads=NT)
    out, lse, *_ = flash_attn_npu_v3.flash_attn_with_kvcache(
        q.to(DEV), kc.to(DEV), vc.to(DEV), cache_seqlens=torch.tensor(L, dtype=torch.int32, device=DEV),
        page_table=bt.to(DEV), cu_seqlens_q=torch.from_numpy(cq).to(DEV), max_seqlen_q=max(lq), causal=True,
        return_softmax_lse=True)
    torch.cuda.synchronize()
    assert_close_out(out, ref_out, dtype)
    assert_close_lse(lse, ref_lse)


# ---- flash_attn_combine ----------------------------------------------------------------------
def test_flash_attn_combine():
    import flash_attn_npu_v3
    print("case flash_attn_combine", flush=True)
    g = _gen(40)
    S, B, Sq, H, Dv = 5, 2, 3, 4, 128
    op = torch.randn((S, B, Sq, H, Dv), generator=g)
    lp = torch.randn((S, B, Sq, H), generator=g) * 3
    lp[1, 0, 0, 0] = -float("inf")          # an empty split
    lp[:, 1, 2, 3] = -float("inf")          # a row with no keys at all
    ref_o, ref_l = orc.combine(op.reshape(S, -1, Dv).numpy(), lp.reshape(S, -1).numpy())
    out, lse = flash_attn_npu_v3.flash_attn_combine(op.to(DEV), lp.to(DEV), out_dtype=torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.cpu().reshape(-1, Dv).numpy(), ref_o, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(lse.cpu().reshape(-1).numpy(), ref_l, rtol=1e-5, atol=1e-5)


# ---- direct C-ABI call (ctypes), no torch operator in between -----------------------------------
def test_capi_direct_dense():
    import ctypes
    from fa_mi355x import capi
    print("case C ABI direct", flush=True)
    g = _gen(50)
    dtype = torch.float16
    B, S, H, D = 1, 257, 4, 128
    q, k, v = (randn((B, S, H, D), dtype, g, "cpu") for _ in range(3))
    ref_out, ref_lse = orc.attention(bits(q).reshape(q.shape), bits(k).reshape(k.shape), bits(v).reshape(v.shape),
                                     dtype=odt(dtype), scale=D ** -0.5, causal=True, nthreads=NT)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    out = torch.empty_like(qd)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=DEV)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    p = capi.new_params(dtype=capi.FA_DTYPE_FP16, batch=B, seqlen_q=S, nheads=H, nheads_k=H, headdim=D,
                        headdim_v=D, seqlen_k=S, batch_cache=B, q=P(qd), q_batch_stride=qd.stride(0),
                        q_row_stride=qd.stride(1), q_head_stride=qd.stride(2), k=P(kd), k_batch_stride=kd.stride(0),
                        k_row_stride=kd.stride(1), k_head_stride=kd.stride(2), v=P(vd), v_batch_stride=vd.stride(0),
                        v_row_stride=vd.stride(1), v_head_stride=vd.stride(2), out=P(out),
                        out_batch_stride=out.stride(0), out_row_stride=out.stride(1), out_head_stride=out.stride(2),
                        softmax_lse=P(lse), softmax_scale=D ** -0.5, is_causal=1)
    st, nbytes = capi.workspace_size(p, capi.FA_KIND_DENSE)
    assert st == capi.FA_OK, capi.last_error()
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=DEV)
    p.workspace, p.workspace_bytes = P(ws), ws.numel()
    st = capi.forward(p, capi.FA_KIND_DENSE, torch.cuda.current_stream().cuda_stream)
    assert st == capi.FA_OK, capi.last_error()
    torch.cuda.synchronize()
    assert_close_out(out, ref_out, dtype)
    assert_close_lse(lse, ref_lse)


def test_errors_raise():
    import flash_attn_npu_v2
    print("case error paths", flush=True)
    q = torch.zeros((1, 4, 8, 128), dtype=torch.bfloat16, device=DEV)
    k = torch.zeros((1, 4, 3, 128), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="divide"):
        flash_attn_npu_v2.flash_attn_func(q, k, k)
    with pytest.raises(RuntimeError, match="dropout"):
        flash_attn_npu_v2.flash_attn_func(q, q, q, dropout_p=0.1)
    with pytest.raises(RuntimeError):
        flash_attn_npu_v2.flash_attn_func(q.float(), q.float(), q.float())
