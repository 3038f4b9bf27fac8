"""GPU parity of the FP8 (e4m3) forward: flash_attn_npu_v3 with
torch.float8_e4m3fn q / k / v (and caches) and q_descale / k_descale /
v_descale, through the torch op and the C ABI, against the CPU oracle
(oracle.fa_oracle.attention_fp8: exact widening of the bytes to bf16, the
blockwise golden per (batch, kv head) with the descaled softmax scale, the
output times v_descale). The reference rejects these arguments
(csrc/arch22/flash_attn_npu_v3/flash_api.cpp:154-156); the semantics are the
v3 API's. Inputs are N(0,1) before quantisation. Tolerances: out (bf16) max-abs 1e-2 times the largest v_descale
plus one bf16 ulp of the reference value, LSE 1e-4 relative, appended
cache bytes bit-exact, and every e4m3 byte decoded exactly."""
import os

import numpy as np
import pytest
import torch

from oracle import fa_oracle as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"
NT = min(16, os.cpu_count() or 1)
F8 = torch.float8_e4m3fn


def fp8(shape, g, amp=1.0):
    return (torch.randn(shape, generator=g) * amp).to(F8)


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


def descales(B, Hk, g, lo=0.5, hi=1.5):
    return [(lo + (hi - lo) * torch.rand((B, Hk), generator=g)).float() for _ in range(3)]


def check(out, lse, ref_o, ref_l, vmax=1.0):
    assert out.dtype == torch.bfloat16
    o = out.float().cpu().numpy()
    err = np.abs(o - ref_o)
    tol = 1e-2 * vmax + np.abs(ref_o) * 2.0 ** -7  # + one bf16 ulp (tests/_util.py ULP)
    assert (err <= tol).all(), f"out max err {err.max():.3e}"
    if lse is not None:
        l = lse.float().cpu().numpy()
        fin = np.isfinite(ref_l)
        assert (np.isfinite(l) == fin).all()
        np.testing.assert_allclose(l[fin], ref_l[fin], rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("path", ["decode", "prefill"])
def test_fp8_every_byte_decodes_exactly(path):
    """One visible key: out = v_descale * v, so every e4m3 code (NaNs left
    out) must come back as its exact value, through the V path of the decode
    and of the prefill kernel (both halves of each 16-byte load)."""
    import flash_attn_npu_v3 as fa3
    print(f"case fp8 every byte {path}", flush=True)
    codes = np.arange(256, dtype=np.uint8)
    codes[[0x7F, 0xFF]] = 0
    want = orc.from_bits(orc.e4m3_to_bf16_bits(codes), orc.BF16).reshape(2, 128)
    v = torch.from_numpy(codes.reshape(2, 1, 1, 128).copy()).view(F8)
    if path == "decode":
        q = torch.zeros((2, 1, 1, 128), dtype=torch.uint8).view(F8)
        kc = torch.zeros((2, 16, 1, 128), dtype=torch.uint8).view(F8)
        vc = torch.zeros((2, 16, 1, 128), dtype=torch.uint8)
        vc[:, 0] = torch.from_numpy(codes.reshape(2, 1, 128).copy())
        out = fa3.flash_attn_with_kvcache(q.to(DEV), kc.to(DEV), vc.view(F8).to(DEV),
                                          cache_seqlens=torch.ones(2, dtype=torch.int32, device=DEV), causal=True)
    else:
        q = torch.zeros((2, 64, 1, 128), dtype=torch.uint8).view(F8)
        k = torch.zeros((2, 1, 1, 128), dtype=torch.uint8).view(F8)
        out = fa3.flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV))
    o = out.float().cpu().numpy()
    assert out.dtype == torch.bfloat16
    for b in range(2):
        assert (o[b, :, 0, :] == want[b][None, :]).all()


@pytest.mark.parametrize("D", [64, 96, 128])
def test_fp8_decode_fused_append_descales(D):
    import flash_attn_npu_v3 as fa3
    print(f"case fp8 decode contiguous fused append D={D}", flush=True)
    g = torch.Generator().manual_seed(D)
    B, H, Hk, S = 3, 8, 2, 1200
    L = torch.tensor([17, 1100, 395], dtype=torch.int32)
    q = fp8((B, 1, H, D), g)
    kc, vc = fp8((B, S, Hk, D), g), fp8((B, S, Hk, D), g)
    kn, vn = fp8((B, 1, Hk, D), g), fp8((B, 1, Hk, D), g)
    qd, kd, vd = descales(B, Hk, g)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    out, lse, *_ = fa3.flash_attn_with_kvcache(q.to(DEV), kc_d, vc_d, k=kn.to(DEV), v=vn.to(DEV),
                                               cache_seqlens=L.to(DEV), q_descale=qd.to(DEV), k_descale=kd.to(DEV),
                                               v_descale=vd.to(DEV), causal=True, return_softmax_lse=True)
    kx, vx = u8(kc).copy(), u8(vc).copy()
    for b in range(B):
        kx[b, L[b]] = u8(kn)[b, 0]
        vx[b, L[b]] = u8(vn)[b, 0]
    assert np.array_equal(u8(kc_d), kx) and np.array_equal(u8(vc_d), vx)
    ro, rl = orc.attention_fp8(u8(q), kx, vx, scale=D ** -0.5, q_descale=qd.numpy(), k_descale=kd.numpy(),
                               v_descale=vd.numpy(), causal=True, seqlens_k=(L + 1).numpy(), nthreads=NT)
    check(out, lse, ro, rl, vmax=float(vd.max()))


@pytest.mark.parametrize("ns", [0, 2])
@pytest.mark.parametrize("page", [64, 48])
def test_fp8_paged_decode_gqa(page, ns):
    # num_splits = 2 forces two key chunks per sequence (the FP8 prefill path)
    import flash_attn_npu_v3 as fa3
    print(f"case fp8 paged decode page={page} num_splits={ns}", flush=True)
    g = torch.Generator().manual_seed(page)
    B, Sq, H, Hk, D = 4, 2, 16, 4, 128
    L = torch.tensor([5, 700, 333, 1500], dtype=torch.int32)
    need = [(int(l) + page - 1) // page for l in L]
    mb = max(need)
    nblocks = sum(need) + 2
    perm = torch.randperm(nblocks, generator=g)
    bt = torch.zeros((B, mb), dtype=torch.int32)
    o = 0
    for b in range(B):
        bt[b, :need[b]] = perm[o:o + need[b]]
        o += need[b]
    kc, vc = fp8((nblocks, page, Hk, D), g), fp8((nblocks, page, Hk, D), g)
    q = fp8((B, Sq, H, D), g)
    qd, kd, vd = descales(B, Hk, g)
    out, lse, *_ = fa3.flash_attn_with_kvcache(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_seqlens=L.to(DEV),
                                               page_table=bt.to(DEV), q_descale=qd.to(DEV), k_descale=kd.to(DEV),
                                               v_descale=vd.to(DEV), causal=True, num_splits=ns,
                                               return_softmax_lse=True)
    # the same keys as a contiguous cache (pages gathered in order)
    kx = u8(kc)[bt.numpy()].reshape(B, mb * page, Hk, D)
    vx = u8(vc)[bt.numpy()].reshape(B, mb * page, Hk, D)
    ro, rl = orc.attention_fp8(u8(q), kx, vx, scale=D ** -0.5, q_descale=qd.numpy(), k_descale=kd.numpy(),
                               v_descale=vd.numpy(), causal=True, seqlens_k=L.numpy(), nthreads=NT)
    check(out, lse, ro, rl, vmax=float(vd.max()))


def test_fp8_paged_decode_many_segments():
    # config-3 regime with fp8: 512 (sequence, kv head) segments and >= 16
    # 64-key tiles per wave worker, so the decode split counts segments
    import flash_attn_npu_v3 as fa3
    print("case fp8 paged decode many segments", flush=True)
    g = torch.Generator().manual_seed(36)
    B, Sq, H, Hk, D, page = 64, 1, 64, 8, 128, 256
    rng = np.random.default_rng(36)
    L = torch.tensor(np.round(np.exp(rng.uniform(np.log(512), np.log(8192), size=B))).astype(np.int32))
    assert B * Hk * int(L.float().mean()) // 64 >= 16 * 1024
    need = [(int(l) + page - 1) // page for l in L]
    mb = max(need)
    nblocks = sum(need) + 2
    perm = torch.randperm(nblocks, generator=g)
    bt = torch.zeros((B, mb), dtype=torch.int32)
    o = 0
    for b in range(B):
        bt[b, :need[b]] = perm[o:o + need[b]]
        o += need[b]
    kc, vc = fp8((nblocks, page, Hk, D), g), fp8((nblocks, page, Hk, D), g)
    q = fp8((B, Sq, H, D), g)
    qd, kd, vd = descales(B, Hk, g)
    out, lse, *_ = fa3.flash_attn_with_kvcache(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_seqlens=L.to(DEV),
                                               page_table=bt.to(DEV), q_descale=qd.to(DEV), k_descale=kd.to(DEV),
                                               v_descale=vd.to(DEV), causal=True, return_softmax_lse=True)
    kx = u8(kc)[bt.numpy()].reshape(B, mb * page, Hk, D)
    vx = u8(vc)[bt.numpy()].reshape(B, mb * page, Hk, D)
    ro, rl = orc.attention_fp8(u8(q), kx, vx, scale=D ** -0.5, q_descale=qd.numpy(), k_descale=kd.numpy(),
                               v_descale=vd.numpy(), causal=True, seqlens_k=L.numpy(), nthreads=NT)
    check(out, lse, ro, rl, vmax=float(vd.max()))


@pytest.mark.parametrize("D,causal,window,softcap", [(64, True, (-1, -1), 0.0), (96, True, (-1, -1), 0.0),
                                                     (128, True, (-1, -1), 0.0), (128, False, (100, 20), 0.0),
                                                     (256, True, (-1, -1), 0.0), (128, True, (-1, -1), 30.0)])
def test_fp8_prefill_dense(D, causal, window, softcap):
    import flash_attn_npu_v3 as fa3
    print(f"case fp8 prefill dense D={D} causal={causal} window={window} softcap={softcap}", flush=True)
    g = torch.Generator().manual_seed(D + int(causal))
    B, Sq, Sk, H, Hk = 2, 300, 420, 8, 2
    q, k, v = fp8((B, Sq, H, D), g), fp8((B, Sk, Hk, D), g), fp8((B, Sk, Hk, D), g)
    qd, kd, vd = descales(B, Hk, g)
    out, lse = fa3.flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal, window_size=window,
                                   softcap=softcap, q_descale=qd.to(DEV), k_descale=kd.to(DEV),
                                   v_descale=vd.to(DEV), return_attn_probs=True)
    ro, rl = orc.attention_fp8(u8(q), u8(k), u8(v), scale=D ** -0.5, q_descale=qd.numpy(), k_descale=kd.numpy(),
                               v_descale=vd.numpy(), causal=causal, window=window, softcap=softcap, nthreads=NT)
    check(out, lse, ro, rl, vmax=float(vd.max()))


def test_fp8_prefill_split_over_keys():
    """Few rows and many keys: the prefill splits the keys and merges fp32
    partials into the bf16 out."""
    import flash_attn_npu_v3 as fa3
    print("case fp8 prefill split", flush=True)
    g = torch.Generator().manual_seed(11)
    B, Sq, Sk, H, Hk, D = 1, 24, 6000, 4, 1, 128
    q, k, v = fp8((B, Sq, H, D), g), fp8((B, Sk, Hk, D), g), fp8((B, Sk, Hk, D), g)
    qd, kd, vd = descales(B, Hk, g)
    out, lse = fa3.flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), causal=True, q_descale=qd.to(DEV),
                                   k_descale=kd.to(DEV), v_descale=vd.to(DEV), return_attn_probs=True)
    ro, rl = orc.attention_fp8(u8(q), u8(k), u8(v), scale=D ** -0.5, q_descale=qd.numpy(), k_descale=kd.numpy(),
                               v_descale=vd.numpy(), causal=True, nthreads=NT)
    check(out, lse, ro, rl, vmax=float(vd.max()))


def test_fp8_varlen():
    import flash_attn_npu_v3 as fa3
    print("case fp8 varlen", flush=True)
    g = torch.Generator().manual_seed(5)
    lq, lk = [37, 190, 1], [80, 190, 333]
    H, Hk, D = 8, 4, 128
    cq = torch.tensor([0] + list(np.cumsum(lq)), dtype=torch.int32)
    ck = torch.tensor([0] + list(np.cumsum(lk)), dtype=torch.int32)
    q, k, v = fp8((sum(lq), H, D), g), fp8((sum(lk), Hk, D), g), fp8((sum(lk), Hk, D), g)
    qd, kd, vd = descales(3, Hk, g)
    out, lse = fa3.flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), cq.to(DEV), ck.to(DEV), max(lq), max(lk),
                                          causal=True, q_descale=qd.to(DEV), k_descale=kd.to(DEV),
                                          v_descale=vd.to(DEV), return_attn_probs=True)
    for b in range(3):
        qs, ks = slice(int(cq[b]), int(cq[b + 1])), slice(int(ck[b]), int(ck[b + 1]))
        ro, rl = orc.attention_fp8(u8(q)[None, qs], u8(k)[None, ks], u8(v)[None, ks], scale=D ** -0.5,
                                   q_descale=qd.numpy()[b:b + 1], k_descale=kd.numpy()[b:b + 1],
                                   v_descale=vd.numpy()[b:b + 1], causal=True, nthreads=NT)
        check(out[qs][None], lse[:, qs][None], ro, rl, vmax=float(vd.max()))


def test_fp8_kvcache_chunked_prefill_append():
    """Many query rows with new tokens: the append runs as its own byte-copy
    kernel, then the prefill kernel reads the fp8 cache."""
    import flash_attn_npu_v3 as fa3
    print("case fp8 kvcache chunked prefill append", flush=True)
    g = torch.Generator().manual_seed(9)
    B, Sn, H, Hk, D, S = 2, 150, 8, 2, 128, 1024
    L = torch.tensor([300, 777], dtype=torch.int32)
    q = fp8((B, Sn, H, D), g)
    kc, vc = fp8((B, S, Hk, D), g), fp8((B, S, Hk, D), g)
    kn, vn = fp8((B, Sn, Hk, D), g), fp8((B, Sn, Hk, D), g)
    qd, kd, vd = descales(B, Hk, g)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    out, lse, *_ = fa3.flash_attn_with_kvcache(q.to(DEV), kc_d, vc_d, k=kn.to(DEV), v=vn.to(DEV),
                                               cache_seqlens=L.to(DEV), q_descale=qd.to(DEV), k_descale=kd.to(DEV),
                                               v_descale=vd.to(DEV), causal=True, return_softmax_lse=True)
    kx, vx = u8(kc).copy(), u8(vc).copy()
    for b in range(B):
        kx[b, L[b]:L[b] + Sn] = u8(kn)[b]
        vx[b, L[b]:L[b] + Sn] = u8(vn)[b]
    assert np.array_equal(u8(kc_d), kx) and np.array_equal(u8(vc_d), vx)
    ro, rl = orc.attention_fp8(u8(q), kx, vx, scale=D ** -0.5, q_descale=qd.numpy(), k_descale=kd.numpy(),
                               v_descale=vd.numpy(), causal=True, seqlens_k=(L + Sn).numpy(), nthreads=NT)
    check(out, lse, ro, rl, vmax=float(vd.max()))


def test_fp8_without_descales_and_rejections():
    import flash_attn_npu_v3 as fa3
    print("case fp8 no descales / rejections", flush=True)
    g = torch.Generator().manual_seed(3)
    q, k, v = fp8((1, 40, 4, 64), g), fp8((1, 90, 2, 64), g), fp8((1, 90, 2, 64), g)
    out, lse = fa3.flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), causal=True, return_attn_probs=True)
    ro, rl = orc.attention_fp8(u8(q), u8(k), u8(v), scale=64 ** -0.5, causal=True, nthreads=NT)
    check(out, lse, ro, rl)
    with pytest.raises(RuntimeError, match="multiple of 16"):
        h = fp8((1, 8, 2, 72), g)
        fa3.flash_attn_func(h.to(DEV), h.to(DEV), h.to(DEV))
    with pytest.raises(RuntimeError, match="dtype"):
        fa3.flash_attn_func(q.to(DEV), k.to(DEV).to(torch.bfloat16), v.to(DEV).to(torch.bfloat16))


def test_fp8_paged_prefill_and_ragged_append():
    """The paged prefill instance (many query rows against a permuted block
    table) and the ragged append (cu_seqlens_q / cu_seqlens_k_new) on FP8
    caches, each against the checker on the equivalent contiguous layout."""
    import flash_attn_npu_v3 as fa3
    print("case fp8 paged prefill + ragged append", flush=True)
    g = torch.Generator().manual_seed(21)
    B, Sq, H, Hk, D, page = 2, 40, 8, 2, 128, 64
    L = torch.tensor([100, 450], dtype=torch.int32)
    need = [(int(l) + page - 1) // page for l in L]
    mb, nblocks = max(need), sum(need) + 1
    perm = torch.randperm(nblocks, generator=g)
    bt = torch.zeros((B, mb), dtype=torch.int32)
    bt[0, :need[0]], bt[1, :need[1]] = perm[:need[0]], perm[need[0]:need[0] + need[1]]
    kc, vc = fp8((nblocks, page, Hk, D), g), fp8((nblocks, page, Hk, D), g)
    q = fp8((B, Sq, H, D), g)
    qd, kd, vd = descales(B, Hk, g)
    out, lse, *_ = fa3.flash_attn_with_kvcache(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_seqlens=L.to(DEV),
                                               page_table=bt.to(DEV), q_descale=qd.to(DEV), k_descale=kd.to(DEV),
                                               v_descale=vd.to(DEV), causal=True, return_softmax_lse=True)
    kx = u8(kc)[bt.numpy()].reshape(B, mb * page, Hk, D)
    vx = u8(vc)[bt.numpy()].reshape(B, mb * page, Hk, D)
    ro, rl = orc.attention_fp8(u8(q), kx, vx, scale=D ** -0.5, q_descale=qd.numpy(), k_descale=kd.numpy(),
                               v_descale=vd.numpy(), causal=True, seqlens_k=L.numpy(), nthreads=NT)
    check(out, lse, ro, rl, vmax=float(vd.max()))

    # ragged queries and ragged new tokens appended into a contiguous FP8 cache
    lq, ln, S = [3, 30], [5, 30], 600
    Lc = torch.tensor([200, 333], dtype=torch.int32)
    cq = torch.tensor([0, 3, 33], dtype=torch.int32)
    cn = torch.tensor([0, 5, 35], dtype=torch.int32)
    q2 = fp8((sum(lq), H, D), g)
    kn, vn = fp8((sum(ln), Hk, D), g), fp8((sum(ln), Hk, D), g)
    kc2, vc2 = fp8((B, S, Hk, D), g), fp8((B, S, Hk, D), g)
    kc2_d, vc2_d = kc2.to(DEV), vc2.to(DEV)
    out2, lse2, *_ = fa3.flash_attn_with_kvcache(q2.to(DEV), kc2_d, vc2_d, k=kn.to(DEV), v=vn.to(DEV),
                                                 cache_seqlens=Lc.to(DEV), cu_seqlens_q=cq.to(DEV),
                                                 cu_seqlens_k_new=cn.to(DEV), max_seqlen_q=max(lq),
                                                 q_descale=qd.to(DEV), k_descale=kd.to(DEV), v_descale=vd.to(DEV),
                                                 causal=True, return_softmax_lse=True)
    kx2, vx2 = u8(kc2).copy(), u8(vc2).copy()
    for b in range(B):
        kx2[b, Lc[b]:Lc[b] + ln[b]] = u8(kn)[cn[b]:cn[b + 1]]
        vx2[b, Lc[b]:Lc[b] + ln[b]] = u8(vn)[cn[b]:cn[b + 1]]
    assert np.array_equal(u8(kc2_d), kx2) and np.array_equal(u8(vc2_d), vx2)
    for b in range(B):
        qs = slice(int(cq[b]), int(cq[b + 1]))
        ro, rl = orc.attention_fp8(u8(q2)[None, qs], kx2[b:b + 1], vx2[b:b + 1], scale=D ** -0.5,
                                   q_descale=qd.numpy()[b:b + 1], k_descale=kd.numpy()[b:b + 1],
                                   v_descale=vd.numpy()[b:b + 1], causal=True,
                                   seqlens_k=np.array([int(Lc[b]) + ln[b]]), nthreads=NT)
        check(out2[qs][None], lse2[:, qs][None], ro, rl, vmax=float(vd.max()))
