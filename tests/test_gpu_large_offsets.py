"""Element offsets beyond 2^31: caches and varlen tensors larger than 4 GiB
(2-byte elements) or 2 GiB (FP8), with the live rows at the high end, so every
address the kernels form past 2^31 elements must be computed in 64 bits.

Paged and contiguous caches: the call on the large cache against the same call
on a compact copy that holds only the live rows, all below 2^31 elements (bit
for bit: the kernels' results do not depend on where a row sits), through the decode kernel, the
forced-split prefill path and a prefill-shaped call with an append and
rotary. Varlen: a dense varlen call over 600 K tokens, its last two sequences
against the CPU oracle."""
import os

import numpy as np
import pytest
import torch

from oracle import fa_oracle as orc
from tests._util import assert_close_lse, assert_close_out, bits, odt

pytestmark = pytest.mark.gpu
DEV = "cuda"
NT = min(16, os.cpu_count() or 1)


def _rand(shape, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(shape, generator=g, device=DEV, dtype=torch.float32)
    return x.to(dtype)


def _same(a, b):
    if a.dtype == torch.float32:
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    return torch.equal(a.view(torch.int16) if a.element_size() == 2 else a.view(torch.uint8),
                       b.view(torch.int16) if b.element_size() == 2 else b.view(torch.uint8))


def _rope(n, rd):
    inv = 1.0 / (10000 ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd))
    ang = torch.arange(n, dtype=torch.float32)[:, None] * inv[None, :]
    return torch.cos(ang).to(torch.bfloat16).to(DEV), torch.sin(ang).to(torch.bfloat16).to(DEV)


@pytest.mark.parametrize("mode", ["decode", "decode_split", "prefill_rotary", "fp8_decode"])
def test_paged_cache_beyond_2g_elements(mode):
    import flash_attn_npu_v3 as fa3
    fp8 = mode == "fp8_decode"
    page, Hk, H, D = 256, 8, 32, 128
    nb = 9000 if not fp8 else 8800          # > 2^31 elements per cache
    assert nb * page * Hk * D > 2 ** 31
    B = 4
    L = [3000, 2100, 700, 4001]
    s_new = {"decode": 1, "decode_split": 1, "prefill_rotary": 64, "fp8_decode": 0}[mode]
    Sq = 64 if mode == "prefill_rotary" else 1
    print(f"case large paged cache {mode}: {nb} blocks of {page} x {Hk} x {D}", flush=True)
    need = [(l + s_new + page - 1) // page for l in L]
    mb = max(need)
    # live blocks at the top of the cache, in a scrambled order
    top = torch.arange(nb - sum(need), nb, dtype=torch.int32)
    top = top[torch.randperm(len(top), generator=torch.Generator().manual_seed(3))]
    bt_big = torch.zeros((B, mb), dtype=torch.int32)
    bt_small = torch.zeros((B, mb), dtype=torch.int32)
    o = 0
    for b in range(B):
        bt_big[b, :need[b]] = top[o:o + need[b]]
        bt_small[b, :need[b]] = torch.arange(o, o + need[b], dtype=torch.int32)
        o += need[b]
    dt = torch.bfloat16
    if fp8:
        kbig = _rand((nb, page, Hk, D), torch.float32, 11).to(torch.float8_e4m3fn)
        vbig = _rand((nb, page, Hk, D), torch.float32, 12).to(torch.float8_e4m3fn)
        q = _rand((B, Sq, H, D), torch.float32, 13).to(torch.float8_e4m3fn)
    else:
        kbig, vbig = _rand((nb, page, Hk, D), dt, 11), _rand((nb, page, Hk, D), dt, 12)
        q = _rand((B, Sq, H, D), dt, 13)
    live = bt_big.flatten()[torch.cat([torch.arange(b * mb, b * mb + need[b]) for b in range(B)])].long().to(DEV)
    ksmall, vsmall = kbig[live].clone(), vbig[live].clone()
    kn = vn = cos = sin = None
    if s_new:
        kn, vn = _rand((B, s_new, Hk, D), dt, 14), _rand((B, s_new, Hk, D), dt, 15)
    if mode == "prefill_rotary":
        cos, sin = _rope(max(L) + s_new + 8, D)
    sl = torch.tensor(L, dtype=torch.int32, device=DEV)
    kw = dict(k=kn, v=vn, rotary_cos=cos, rotary_sin=sin, cache_seqlens=sl, causal=True,
              num_splits=3 if mode == "decode_split" else 0, return_softmax_lse=True)
    if fp8:
        ds = torch.ones((B, Hk), dtype=torch.float32, device=DEV)
        kw.update(q_descale=ds, k_descale=ds * 0.5, v_descale=ds * 1.5)
    o1, l1, *_ = fa3.flash_attn_with_kvcache(q, kbig, vbig, page_table=bt_big.to(DEV), **kw)
    o0, l0, *_ = fa3.flash_attn_with_kvcache(q, ksmall, vsmall, page_table=bt_small.to(DEV), **kw)
    torch.cuda.synchronize()
    assert _same(o0, o1) and _same(l0, l1), "large-cache result differs from the compact-cache result"
    assert _same(kbig[live], ksmall) and _same(vbig[live], vsmall), "appended rows differ"
    assert torch.isfinite(o1.float()).all()


def test_contiguous_cache_beyond_2g_elements():
    import flash_attn_npu_v2
    B, cap, Hk, H, D = 4, 700000, 8, 32, 128
    assert 3 * cap * Hk * D > 2 ** 31  # the last sequence's rows start past 2^31 elements
    print(f"case large contiguous cache {B} x {cap} x {Hk} x {D}", flush=True)
    dt = torch.bfloat16
    kbig, vbig = _rand((B, cap, Hk, D), dt, 21), _rand((B, cap, Hk, D), dt, 22)
    L = [1000, 300, 5000, 4000]
    cap2 = max(L) + 8                        # the compact copy: every offset below 2^31
    ksmall, vsmall = kbig[:, :cap2].clone(), vbig[:, :cap2].clone()
    q = _rand((B, 1, H, D), dt, 23)
    kn, vn = _rand((B, 1, Hk, D), dt, 24), _rand((B, 1, Hk, D), dt, 25)
    sl = torch.tensor(L, dtype=torch.int32, device=DEV)
    for ns in (0, 3):
        o1, l1 = flash_attn_npu_v2.flash_attn_with_kvcache(q, kbig, vbig, k=kn, v=vn, cache_seqlens=sl, causal=True,
                                                          num_splits=ns, return_softmax_lse=True)
        o0, l0 = flash_attn_npu_v2.flash_attn_with_kvcache(q, ksmall, vsmall, k=kn, v=vn, cache_seqlens=sl,
                                                          causal=True, num_splits=ns, return_softmax_lse=True)
        torch.cuda.synchronize()
        assert _same(o0, o1) and _same(l0, l1), f"num_splits={ns}: large-cache result differs"
        assert _same(kbig[:, :cap2], ksmall) and _same(vbig[:, :cap2], vsmall), "appended rows differ"


def test_varlen_beyond_2g_elements():
    import flash_attn_npu_v2
    H, Hk, D, n, ln = 32, 8, 128, 500, 1200
    T = n * ln
    assert T * H * D > 2 ** 31
    print(f"case large varlen {n} x {ln} tokens, H{H}/{Hk} D{D}", flush=True)
    dt = torch.bfloat16
    q, k, v = _rand((T, H, D), dt, 31), _rand((T, Hk, D), dt, 32), _rand((T, Hk, D), dt, 33)
    cu = torch.arange(n + 1, dtype=torch.int32, device=DEV) * ln
    out, lse, _ = flash_attn_npu_v2.flash_attn_varlen_func(q, k, v, cu, cu, ln, ln, causal=True,
                                                          return_attn_probs=True)
    torch.cuda.synchronize()
    # the last two sequences against the oracle (host copies of their rows)
    r0 = (n - 2) * ln
    qs, ks, vs = (x[r0:].cpu() for x in (q, k, v))
    cus = np.array([0, ln, 2 * ln], np.int32)
    ro, rl = orc.attention(bits(qs), bits(ks), bits(vs), dtype=odt(dt), scale=D ** -0.5, causal=True,
                           cu_seqlens_q=cus, cu_seqlens_k=cus, max_seqlen_q=ln, nthreads=NT)
    assert_close_out(out[r0:], ro, dt)
    assert_close_lse(lse[:, r0:], rl)


def test_varlen_backward_beyond_2g_elements():
    """The backward over 600 K tokens (q, dout, dq past 2^31 elements): the
    last two sequences' gradients against the float64 oracle."""
    import flash_attn_npu_v2
    from tests import test_gpu_bwd as tb
    from oracle import fa_bwd_oracle as bo
    H, Hk, D, n, ln = 32, 8, 128, 500, 1200
    T = n * ln
    assert T * H * D > 2 ** 31
    print(f"case large varlen backward {n} x {ln} tokens, H{H}/{Hk} D{D}", flush=True)
    dt = torch.bfloat16
    u = lambda shape, seed: (2.0 * torch.rand(shape, generator=torch.Generator(device=DEV).manual_seed(seed),
                                              device=DEV) - 1.0).to(dt)
    q, k, v, do = u((T, H, D), 41), u((T, Hk, D), 42), u((T, Hk, D), 43), u((T, H, D), 44)
    cu = torch.arange(n + 1, dtype=torch.int32, device=DEV) * ln
    qd, kd, vd = (x.requires_grad_(True) for x in (q, k, v))
    out, lse, _ = flash_attn_npu_v2.flash_attn_varlen_func(qd, kd, vd, cu, cu, ln, ln, causal=True,
                                                          return_attn_probs=True)
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), do)
    torch.cuda.synchronize()
    r0 = (n - 2) * ln
    cus = np.array([0, ln, 2 * ln], np.int32)
    f = lambda x: x[r0:].detach().float().cpu().numpy()
    rq, rk, rv = bo.attention_bwd(f(q), f(k), f(v), f(do), lse[:, r0:].detach().cpu().numpy(), scale=D ** -0.5,
                                  softcap=0.0, causal=True, window=(-1, -1), cu_seqlens_q=cus, cu_seqlens_k=cus)
    tb.check("dq", dq[r0:], rq)
    tb.check("dk", dk[r0:], rk)
    tb.check("dv", dv[r0:], rv)
