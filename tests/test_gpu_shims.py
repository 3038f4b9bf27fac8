"""The reference-side module shims flash_attn_npu_arch22_v2 / _v3 (the
pybind11 module names and positional signatures the reference's Python layer
calls: csrc/arch22/flash_attn_npu_v2/flash_api.cpp:1301-1309,
csrc/arch22/flash_attn_npu_v3/flash_api.cpp:816-822, called at
flash_attn_npu_v3/interface_arch22.py:111-146) give bit for bit the results of
the public API."""
import numpy as np
import pytest
import torch

from tests._util import bits, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _eq(a, b):
    if a.dtype == torch.float32:
        return np.array_equal(a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32))
    return np.array_equal(bits(a), bits(b))


def test_v2_shim_positional():
    import flash_attn_npu_arch22_v2 as m
    import flash_attn_npu_v2 as api
    print("case shim v2", flush=True)
    g = torch.Generator().manual_seed(900)
    dt = torch.bfloat16
    q, k, v = randn((2, 70, 8, 128), dt, g, DEV), randn((2, 90, 2, 128), dt, g, DEV), randn((2, 90, 2, 128), dt, g, DEV)
    s = 128 ** -0.5
    # fwd(q, k, v, out_, alibi, p_dropout, scale, causal, wl, wr, softcap, return_softmax, gen)
    out_ = torch.empty_like(q)
    o, l, p, rng = m.fwd(q, k, v, out_, None, 0.0, s, True, -1, 0, 0.0, False, None)
    ro, rl, _ = api.flash_attn_func(q, k, v, causal=True, return_attn_probs=True)
    assert o is out_ and _eq(o, ro) and _eq(l, rl) and p.numel() == 0 and rng.numel() == 0
    # bwd(dout, q, k, v, out, lse, dq_, dk_, dv_, alibi, p_dropout, scale, causal, wl, wr, softcap, det, gen, rng)
    do = randn((2, 70, 8, 128), dt, g, DEV)
    dq, dk, dv, sd = m.bwd(do, q, k, v, o, l, None, None, None, None, 0.0, s, True, -1, 0, 0.0, False, None, None)
    qd, kd, vd = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
    ref = torch.autograd.grad(api.flash_attn_func(qd, kd, vd, causal=True), (qd, kd, vd), do)
    assert all(_eq(a, b) for a, b in zip((dq, dk, dv), ref)) and sd.shape == (2, 8, 70)
    # varlen_fwd(q, k, v, out_, cu_q, cu_k, seqused_k, leftpad_k, block_table, alibi, max_q, max_k, p_dropout,
    #            scale, zero_tensors, causal, wl, wr, softcap, return_softmax, gen)
    cu = torch.tensor([0, 30, 90], dtype=torch.int32, device=DEV)
    qv, kv = randn((90, 8, 128), dt, g, DEV), randn((90, 2, 128), dt, g, DEV)
    o, l, _, _ = m.varlen_fwd(qv, kv, kv, None, cu, cu, None, None, None, None, 60, 60, 0.0, s, False, True, -1, 0, 0.0,
                              False, None)
    ro, rl, _ = api.flash_attn_varlen_func(qv, kv, kv, cu, cu, 60, 60, causal=True, return_attn_probs=True)
    assert _eq(o, ro) and _eq(l, rl)
    # varlen_bwd(dout, q, k, v, out, lse, dq_, dk_, dv_, cu_q, cu_k, alibi, max_q, max_k, p_dropout, scale,
    #            zero_tensors, causal, wl, wr, softcap, det, gen, rng)
    dov = randn((90, 8, 128), dt, g, DEV)
    dq_ = torch.empty_like(qv)
    dq, dk, dv, _ = m.varlen_bwd(dov, qv, kv, kv, o, l, dq_, None, None, cu, cu, None, 60, 60, 0.0, s, False, True,
                                 -1, 0, 0.0, False, None, None)
    qd, kd = qv.detach().clone().requires_grad_(True), kv.detach().clone().requires_grad_(True)
    vd = kv.detach().clone().requires_grad_(True)
    ref = torch.autograd.grad(api.flash_attn_varlen_func(qd, kd, vd, cu, cu, 60, 60, causal=True), (qd, kd, vd), dov)
    assert dq is dq_ and all(_eq(a, b) for a, b in zip((dq, dk, dv), ref))
    # fwd_kvcache(q, kcache, vcache, k_, v_, seqlens_k, cos, sin, cache_batch_idx, leftpad_k, block_table, alibi,
    #             out_, scale, causal, wl, wr, softcap, rotary_interleaved, num_splits)
    qk = randn((3, 1, 32, 128), dt, g, DEV)
    kc, vc = randn((3, 512, 8, 128), dt, g, DEV), randn((3, 512, 8, 128), dt, g, DEV)
    kn, vn = randn((3, 1, 8, 128), dt, g, DEV), randn((3, 1, 8, 128), dt, g, DEV)
    sl = torch.tensor([10, 300, 511], dtype=torch.int32, device=DEV)
    kc2, vc2 = kc.clone(), vc.clone()
    o, l = m.fwd_kvcache(qk, kc, vc, kn, vn, sl, None, None, None, None, None, None, None, s, True, -1, 0, 0.0, True, 0)
    ro, rl = api.flash_attn_with_kvcache(qk, kc2, vc2, k=kn, v=vn, cache_seqlens=sl, causal=True,
                                         return_softmax_lse=True)
    assert _eq(o, ro) and _eq(l, rl) and _eq(kc, kc2) and _eq(vc, vc2)


def test_v3_shim_positional():
    import flash_attn_npu_arch22_v3 as m
    import flash_attn_npu_v3 as api
    print("case shim v3", flush=True)
    g = torch.Generator().manual_seed(901)
    dt = torch.float16
    s = 128 ** -0.5
    q, k, v = randn((2, 70, 8, 128), dt, g, DEV), randn((2, 90, 2, 128), dt, g, DEV), randn((2, 90, 2, 128), dt, g, DEV)
    none8 = (None,) * 8

    def call(q, k, v, k_new=None, v_new=None, cu_q=None, cu_k=None, seqused_k=None, max_q=None, max_k=None,
             page_table=None, causal=True, md=None, num_splits=1, qv=None, pack_gqa=None):
        # the positional order of flash_attn_npu_v3/interface_arch22.py:111-146
        return m.fwd(q, k, v, k_new, v_new, qv, None, cu_q, cu_k, None, None, seqused_k, max_q, max_k, page_table,
                     None, None, None, None, None, None, None, None, s, causal, -1, -1, 0, 0.0, True, md, num_splits,
                     pack_gqa, 0)

    o, l, oa, la = call(q, k, v)
    ro, rl = api.flash_attn_func(q, k, v, causal=True, return_attn_probs=True)
    assert _eq(o, ro) and _eq(l, rl) and oa.numel() == 0 and la.numel() == 0
    cu = torch.tensor([0, 30, 90], dtype=torch.int32, device=DEV)
    qv, kv = randn((90, 8, 128), dt, g, DEV), randn((90, 2, 128), dt, g, DEV)
    o, l, _, _ = call(qv, kv, kv, cu_q=cu, cu_k=cu, max_q=60, max_k=60)
    ro, rl = api.flash_attn_varlen_func(qv, kv, kv, cu, cu, 60, 60, causal=True, return_attn_probs=True)
    assert _eq(o, ro) and _eq(l, rl)
    qk = randn((3, 2, 32, 128), dt, g, DEV)
    kc, vc = randn((3, 512, 8, 128), dt, g, DEV), randn((3, 512, 8, 128), dt, g, DEV)
    kn, vn = randn((3, 2, 8, 128), dt, g, DEV), randn((3, 2, 8, 128), dt, g, DEV)
    sl = torch.tensor([10, 300, 500], dtype=torch.int32, device=DEV)
    kc2, vc2 = kc.clone(), vc.clone()
    md = m.get_scheduler_metadata(3, 2, 512, 32, 8, 128, 128, dt, sl, None, None, None, None, None, None, 0, True,
                                  -1, -1, 0, False, 0, None, 0)
    o, l, _, _ = call(qk, kc, vc, k_new=kn, v_new=vn, seqused_k=sl, md=md, num_splits=0)
    ro, rl, *_ = api.flash_attn_with_kvcache(qk, kc2, vc2, k=kn, v=vn, cache_seqlens=sl, causal=True,
                                             return_softmax_lse=True)
    assert _eq(o, ro) and _eq(l, rl) and _eq(kc, kc2) and _eq(vc, vc2)
    # qv (the reference's q_v_ argument) on a decode call, and pack_gqa = False
    qd1, qvd = randn((3, 1, 32, 128), dt, g, DEV), randn((3, 1, 32, 128), dt, g, DEV)
    o, l, _, _ = call(qd1, kc, vc, seqused_k=sl, qv=qvd, num_splits=0)
    ro, rl, *_ = api.flash_attn_with_kvcache(qd1, kc, vc, qv=qvd, cache_seqlens=sl, softmax_scale=s, causal=True,
                                             return_softmax_lse=True)
    assert _eq(o, ro) and _eq(l, rl)
    o, l, _, _ = call(q, k, v, pack_gqa=False)
    ro, rl = api.flash_attn_func(q, k, v, causal=True, pack_gqa=False, return_attn_probs=True)
    assert _eq(o, ro) and _eq(l, rl)
    # bwd(dout, q, k, v, out, lse, dq_, dk_, dv_, cu_q, cu_k, seqused_q, seqused_k, max_q, max_k, scale, causal,
    #     wl, wr, softcap, deterministic, sm_margin)
    o, l, _, _ = call(q, k, v)
    do = randn((2, 70, 8, 128), dt, g, DEV)
    dq, dk, dv, sd = m.bwd(do, q, k, v, o, l, None, None, None, None, None, None, None, None, None, s, True, -1, -1,
                           0.0, False, 0)
    qd, kd, vd = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
    ref = torch.autograd.grad(api.flash_attn_func(qd, kd, vd, causal=True), (qd, kd, vd), do)
    assert all(_eq(a, b) for a, b in zip((dq, dk, dv), ref))
    op = torch.randn((3, 2, 5, 4, 128), generator=g).to(DEV)
    lp = torch.randn((3, 2, 5, 4), generator=g).to(DEV)
    o1, l1 = m.fwd_combine(op, lp, None, torch.bfloat16)
    o2, l2 = api.flash_attn_combine(op, lp, out_dtype=torch.bfloat16)
    assert _eq(o1, o2) and _eq(l1, l2)
