"""GPU parity of two v3 API parameters the reference declares and does not
implement (flash_attn_npu_v3/interface_arch22.py:940-962; its kernel ignores
q_v_, csrc/arch22/flash_attn_npu_v3/flash_api.cpp:66, and rejects pack_gqa =
True, :162), with FlashAttention-3's semantics:

  * qv: scores = softmax_scale * (q . k + qv . v), default scale
    (headdim + headdim_v) ** -0.5. The decode kernel takes it directly; the
    dense / varlen entry points run it as one attention over the concatenated
    head dims. Checked against the CPU oracle's qv (pinned in
    tests/test_oracle.py against that concatenation and a float64 brute force).
  * pack_gqa = False: each query head gets its own row tiles. Checked against
    the oracle and against pack_gqa = True. The two agree to rounding, not bit
    for bit: a wave rescales its rows' running maxima together when any row
    needs it, so a row's rounding depends on the rows sharing its wave."""
import os

import numpy as np
import pytest
import torch

from oracle import fa_oracle as orc
from tests._util import assert_close_lse, assert_close_out, bits, odt, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
NT = min(16, os.cpu_count() or 1)


def _kvcache_case(*, B, Sq, H, Hk, D, dtype, L, capacity=0, page=0, new=0, window=(-1, -1), ragged=None,
                  pack_gqa=None, seed=0, with_qv=True, softcap=0.0):
    import flash_attn_npu_v3
    print(f"case qv kvcache B{B} Sq{Sq} H{H}/{Hk} D{D} page{page} new{new} win{window} ragged{ragged} "
          f"pack{pack_gqa} qv{with_qv} softcap{softcap}", flush=True)
    g = torch.Generator().manual_seed(seed)
    if ragged is not None:
        cu_q = np.concatenate([[0], np.cumsum(ragged)]).astype(np.int32)
        q = randn((int(cu_q[-1]), H, D), dtype, g, "cpu")
    else:
        cu_q = None
        q = randn((B, Sq, H, D), dtype, g, "cpu")
    qv = randn(q.shape, dtype, g, "cpu") if with_qv else None
    L = np.asarray(L, np.int32)
    kn = vn = None
    if new:
        kn = randn((B, new, Hk, D), dtype, g, "cpu")
        vn = randn((B, new, Hk, D), dtype, g, "cpu")
    bt = None
    if page:
        need = [(int(L[b]) + new + page - 1) // page for b in range(B)]
        nblocks = sum(need) + 2
        perm = torch.randperm(nblocks, generator=g).to(torch.int32)
        bt = torch.zeros((B, max(need)), dtype=torch.int32)
        o = 0
        for b in range(B):
            bt[b, :need[b]] = perm[o:o + need[b]]
            o += need[b]
        kc, vc = randn((nblocks, page, Hk, D), dtype, g, "cpu"), randn((nblocks, page, Hk, D), dtype, g, "cpu")
    else:
        kc, vc = randn((B, capacity, Hk, D), dtype, g, "cpu"), randn((B, capacity, Hk, D), dtype, g, "cpu")
    ro, rl, rk, _ = orc.kvcache_forward_v3(
        bits(q), bits(kc), bits(vc), dtype=odt(dtype), cache_seqlens=L,
        k=None if kn is None else bits(kn), v=None if vn is None else bits(vn),
        block_table=None if bt is None else bt.numpy(), causal=True, window=window, softcap=softcap,
        cu_seqlens_q=cu_q, max_seqlen_q=None if ragged is None else int(max(ragged)),
        qv=None if qv is None else bits(qv), nthreads=NT)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    out, lse, *_ = flash_attn_npu_v3.flash_attn_with_kvcache(
        q.to(DEV), kc_d, vc_d, k=None if kn is None else kn.to(DEV), v=None if vn is None else vn.to(DEV),
        qv=None if qv is None else qv.to(DEV),
        cache_seqlens=torch.from_numpy(L).to(DEV), page_table=None if bt is None else bt.to(DEV),
        cu_seqlens_q=None if cu_q is None else torch.from_numpy(cu_q).to(DEV),
        max_seqlen_q=None if ragged is None else int(max(ragged)), causal=True, window_size=window,
        softcap=softcap, pack_gqa=pack_gqa, return_softmax_lse=True)
    torch.cuda.synchronize()
    assert_close_out(out, ro, dtype)
    assert_close_lse(lse, rl)
    assert np.array_equal(bits(kc_d), rk), "cache after the append differs"
    return out, lse


QV_KV = [
    dict(B=3, Sq=1, H=16, Hk=4, D=128, dtype=torch.bfloat16, L=[700, 31, 2000], capacity=2048, new=1),
    dict(B=2, Sq=4, H=8, Hk=2, D=128, dtype=torch.float16, L=[300, 900], page=64, window=(50, 0)),
    dict(B=3, Sq=2, H=8, Hk=2, D=128, dtype=torch.bfloat16, L=[100, 500, 64], capacity=512, ragged=[2, 1, 2]),
    dict(B=2, Sq=1, H=8, Hk=1, D=96, dtype=torch.bfloat16, L=[1000, 77], capacity=1024, new=1),
    dict(B=2, Sq=4, H=32, Hk=8, D=128, dtype=torch.bfloat16, L=[400, 1500], page=256, pack_gqa=False),
    # soft capping: qv . v enters the capped score
    dict(B=3, Sq=1, H=16, Hk=4, D=128, dtype=torch.bfloat16, L=[900, 40, 1700], capacity=2048, new=1, softcap=5.0),
    dict(B=2, Sq=2, H=8, Hk=2, D=64, dtype=torch.float16, L=[333, 1200], page=64, window=(100, 0), softcap=2.0),
]


@pytest.mark.parametrize("case", QV_KV, ids=[str(i) for i in range(len(QV_KV))])
def test_qv_kvcache_decode_vs_oracle(case):
    _kvcache_case(seed=500, **case)


@pytest.mark.parametrize("ns", [0, 3])
def test_qv_decode_with_alibi_through_the_op(ns):
    # the v3 Python API has no alibi_slopes; the operator does (the decode
    # kernel's qv instance forms its scores explicitly, ALiBi included). A
    # forced split count keeps a qv call on the decode kernel (only it forms
    # the qv term).
    from fa_mi355x import ops
    print(f"case qv decode + ALiBi (op), num_splits={ns}", flush=True)
    g = torch.Generator().manual_seed(560)
    B, H, Hk, D, dtype = 3, 16, 4, 128, torch.bfloat16
    L = np.array([1200, 77, 600], np.int32)
    q, qv = randn((B, 2, H, D), dtype, g, "cpu"), randn((B, 2, H, D), dtype, g, "cpu")
    kc, vc = randn((B, 1536, Hk, D), dtype, g, "cpu"), randn((B, 1536, Hk, D), dtype, g, "cpu")
    slopes = (2.0 ** (-8.0 * (torch.arange(H) + 1) / H)).float()
    scale = (2 * D) ** -0.5
    ro, rl, _, _ = orc.kvcache_forward_v3(bits(q), bits(kc), bits(vc), dtype=orc.BF16, cache_seqlens=L,
                                          softmax_scale=scale, causal=True, alibi=slopes.numpy(), qv=bits(qv),
                                          nthreads=NT)
    out, lse = ops.fwd_kvcache_v3(q.to(DEV), kc.to(DEV), vc.to(DEV), None, None, torch.from_numpy(L).to(DEV), None,
                                  None, None, None, None, slopes.to(DEV), None, None, 0, None, scale, True, -1, 0, 0,
                                  0.0, True, ns, None, None, None, None, qv.to(DEV), None)
    torch.cuda.synchronize()
    assert_close_out(out, ro, dtype)
    assert_close_lse(lse, rl)


def test_qv_rejected_where_the_decode_kernel_does_not_run():
    import flash_attn_npu_v3
    q = torch.randn(1, 64, 8, 64, device=DEV, dtype=torch.bfloat16)
    kc = torch.randn(1, 128, 2, 64, device=DEV, dtype=torch.bfloat16)
    L = torch.tensor([100], dtype=torch.int32, device=DEV)
    print("case qv on a prefill-shaped kvcache call", flush=True)
    with pytest.raises(RuntimeError, match="qv is supported where the decode kernel runs"):
        flash_attn_npu_v3.flash_attn_with_kvcache(q, kc, kc.clone(), qv=torch.randn_like(q), cache_seqlens=L)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_qv_dense_and_varlen_vs_oracle(dtype):
    import flash_attn_npu_v3
    print(f"case qv dense/varlen {dtype}", flush=True)
    g = torch.Generator().manual_seed(510)
    B, S, H, Hk, D = 2, 300, 8, 2, 64
    q, qv = randn((B, S, H, D), dtype, g, "cpu"), randn((B, S, H, D), dtype, g, "cpu")
    k, v = randn((B, S, Hk, D), dtype, g, "cpu"), randn((B, S, Hk, D), dtype, g, "cpu")
    ro, rl = orc.attention(bits(q), bits(k), bits(v), dtype=odt(dtype), scale=(2 * D) ** -0.5, causal=True,
                           qv=bits(qv), nthreads=NT)
    out, lse = flash_attn_npu_v3.flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), qv=qv.to(DEV), causal=True,
                                                 return_attn_probs=True)
    assert_close_out(out, ro, dtype)
    assert_close_lse(lse, rl)
    # varlen: the same rows as two packed sequences
    cu = torch.tensor([0, S, 2 * S], dtype=torch.int32)
    outv, lsev = flash_attn_npu_v3.flash_attn_varlen_func(
        q.reshape(B * S, H, D).to(DEV), k.reshape(B * S, Hk, D).to(DEV), v.reshape(B * S, Hk, D).to(DEV),
        cu.to(DEV), cu.to(DEV), S, S, qv=qv.reshape(B * S, H, D).to(DEV), causal=True, return_attn_probs=True)
    assert_close_out(outv.reshape(B, S, H, D), ro, dtype)
    assert_close_lse(lsev.reshape(H, B, S).permute(1, 0, 2), rl)


def test_qv_dense_backward_vs_fp32_reference():
    import flash_attn_npu_v3
    print("case qv dense backward", flush=True)
    g = torch.Generator().manual_seed(520)
    B, S, H, Hk, D, dtype = 1, 96, 4, 2, 64, torch.bfloat16
    ts = [randn(s, dtype, g, "cpu") for s in ((B, S, H, D), (B, S, H, D), (B, S, Hk, D), (B, S, Hk, D))]
    dout = randn((B, S, H, D), dtype, g, "cpu")
    dev = [t.to(DEV).requires_grad_() for t in ts]
    out = flash_attn_npu_v3.flash_attn_func(dev[0], dev[2], dev[3], qv=dev[1], causal=True)
    out.backward(dout.to(DEV))
    # fp32 reference on the CPU: scores = (q.k + qv.v) * scale, GQA by repetition
    ref = [t.float().requires_grad_() for t in ts]
    q, qv, k, v = ref
    kr, vr = k.repeat_interleave(H // Hk, 2), v.repeat_interleave(H // Hk, 2)
    s = (torch.einsum("bihd,bjhd->bhij", q, kr) + torch.einsum("bihd,bjhd->bhij", qv, vr)) * (2 * D) ** -0.5
    s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    o = torch.einsum("bhij,bjhd->bihd", torch.softmax(s, -1), vr)
    o.backward(dout.float())
    assert (out.detach().float().cpu() - o.detach()).abs().max() < 2e-2
    for name, got, want in zip(("dq", "dqv", "dk", "dv"), dev, ref):
        gr, wr = got.grad.float().cpu(), want.grad
        rel = float((gr - wr).norm() / wr.norm())
        assert rel < 2e-2, f"{name} relative error {rel:.3e}"


# ---- pack_gqa = False ------------------------------------------------------------------------
def _agree(packed, unpacked, dtype):
    """(out, lse) of the two layouts: out within the output tolerance plus
    one ulp of the value (both are rounded to 16 bits), lse within the
    lse tolerance."""
    assert_close_out(unpacked[0], bits(packed[0]), dtype)
    assert_close_lse(unpacked[1], packed[1].float().cpu().numpy())


def test_pack_gqa_false_kvcache_decode_vs_oracle_and_packed():
    base = dict(B=4, Sq=1, H=32, Hk=8, D=128, dtype=torch.bfloat16, L=[3000, 70, 1200, 4000], capacity=4096,
                new=1, with_qv=False)
    o1, l1 = _kvcache_case(seed=530, pack_gqa=False, **base)
    o2, l2 = _kvcache_case(seed=530, pack_gqa=True, **base)
    _agree((o2, l2), (o1, l1), torch.bfloat16)


@pytest.mark.parametrize("fp8", [False, True])
def test_pack_gqa_false_dense_prefill(fp8):
    from fa_mi355x import ops
    print(f"case pack_gqa dense prefill fp8={fp8}", flush=True)
    g = torch.Generator().manual_seed(540)
    B, S, H, Hk, D = 2, 384, 16, 4, 128
    q, k, v = (randn(s, torch.bfloat16, g, "cpu") for s in ((B, S, H, D), (B, S, Hk, D), (B, S, Hk, D)))
    desc = (None, None, None)
    if fp8:
        q, k, v = (t.to(torch.float8_e4m3fn) for t in (q, k, v))
        desc = tuple((torch.rand((B, Hk), generator=g) + 0.5).to(DEV) for _ in range(3))
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    alibi = None if fp8 else (2.0 ** (-8.0 * (torch.arange(H) + 1) / H)).float().to(DEV)
    res = [ops.fwd(q, k, v, alibi, 0.0, D ** -0.5, True, 200, 0, 0.0, 0, *desc, 1, None, pack)
           for pack in (True, False)]
    torch.cuda.synchronize()
    _agree(res[0], res[1], torch.bfloat16)
    if not fp8:
        ro, rl = orc.attention(bits(q), bits(k), bits(v), dtype=orc.BF16, scale=D ** -0.5, causal=True,
                               window=(200, 0), alibi=alibi.cpu().numpy(), nthreads=NT)
        assert_close_out(res[1][0], ro, torch.bfloat16)
        assert_close_lse(res[1][1], rl)


def test_pack_gqa_false_varlen():
    import flash_attn_npu_v3
    print("case pack_gqa varlen", flush=True)
    g = torch.Generator().manual_seed(550)
    H, Hk, D = 8, 2, 64
    lens = [130, 7, 260]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32).to(DEV)
    T = sum(lens)
    q, k, v = (randn(s, torch.float16, g, "cpu").to(DEV) for s in ((T, H, D), (T, Hk, D), (T, Hk, D)))
    outs = [flash_attn_npu_v3.flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), causal=True,
                                                     num_splits=1, pack_gqa=pack, return_attn_probs=True)
            for pack in (None, False)]
    torch.cuda.synchronize()
    _agree(outs[0], outs[1], torch.float16)
    ro, rl = orc.attention(bits(q), bits(k), bits(v), dtype=orc.FP16, scale=D ** -0.5, causal=True,
                           cu_seqlens_q=cu.cpu().numpy(), cu_seqlens_k=cu.cpu().numpy(), max_seqlen_q=max(lens),
                           nthreads=NT)
    assert_close_out(outs[1][0], ro, torch.float16)
    assert_close_lse(outs[1][1], rl)
