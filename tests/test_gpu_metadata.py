"""scheduler_metadata on the GPU, mirroring the reference's four metadata
tests (tests/test_flash_attn_npu_v3_metadata.py:214-443): flash_attn_func
(BSND), flash_attn_varlen_func (TND) and flash_attn_with_kvcache (BSND paged,
TND paged) given get_scheduler_metadata's plan give bit for bit the result of
the same call without it (with the metadata's split count), within tolerance
of the CPU oracle; a call the metadata does not describe raises."""
import os

import numpy as np
import pytest
import torch

from oracle import fa_oracle as orc
from tests._util import assert_close_lse, assert_close_out, bits, odt, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
NT = min(16, os.cpu_count() or 1)


def _same(a, b):
    return np.array_equal(bits(a) if a.dtype != torch.float32 else a.cpu().numpy().view(np.uint32),
                          bits(b) if b.dtype != torch.float32 else b.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("causal,num_splits", [(True, 0), (False, 1), (True, 3)])
def test_flash_attn_func_metadata_bsnd(causal, num_splits):
    from flash_attn_npu_v3 import flash_attn_func, get_scheduler_metadata
    print(f"case metadata func causal={causal} splits={num_splits}", flush=True)
    g = torch.Generator().manual_seed(700)
    B, Sq, Sk, H, Hk, D, dt = 2, 200, 333, 8, 2, 128, torch.bfloat16
    q, k, v = randn((B, Sq, H, D), dt, g, DEV), randn((B, Sk, Hk, D), dt, g, DEV), randn((B, Sk, Hk, D), dt, g, DEV)
    md = get_scheduler_metadata(B, Sq, Sk, H, Hk, D, torch.full((B,), Sk, dtype=torch.int32, device=DEV),
                                qkv_dtype=dt, causal=causal, num_splits=num_splits)
    o1, l1 = flash_attn_func(q, k, v, causal=causal, num_splits=1, return_attn_probs=True, scheduler_metadata=md)
    o0, l0 = flash_attn_func(q, k, v, causal=causal, num_splits=num_splits, return_attn_probs=True)
    torch.cuda.synchronize()
    assert _same(o0, o1) and _same(l0, l1), "metadata changed the result"
    ro, rl = orc.attention(bits(q), bits(k), bits(v), dtype=odt(dt), scale=D ** -0.5, causal=causal, nthreads=NT)
    assert_close_out(o1, ro, dt)
    assert_close_lse(l1, rl)
    with pytest.raises(RuntimeError, match="different call"):
        flash_attn_func(q, k, v, causal=not causal, scheduler_metadata=md)
    with pytest.raises(RuntimeError, match="different call"):
        flash_attn_func(q[:, :, :4], k[:, :, :1], v[:, :, :1], causal=causal, scheduler_metadata=md)


def test_flash_attn_varlen_func_metadata_tnd():
    from flash_attn_npu_v3 import flash_attn_varlen_func, get_scheduler_metadata
    print("case metadata varlen", flush=True)
    g = torch.Generator().manual_seed(701)
    H, Hk, D, dt = 8, 2, 128, torch.float16
    lq, lk = [37, 1, 300, 128], [37, 90, 300, 1000]
    cq = torch.tensor(np.concatenate([[0], np.cumsum(lq)]), dtype=torch.int32, device=DEV)
    ck = torch.tensor(np.concatenate([[0], np.cumsum(lk)]), dtype=torch.int32, device=DEV)
    q, k, v = randn((sum(lq), H, D), dt, g, DEV), randn((sum(lk), Hk, D), dt, g, DEV), randn((sum(lk), Hk, D), dt, g, DEV)
    md = get_scheduler_metadata(4, max(lq), max(lk), H, Hk, D, torch.tensor(lk, dtype=torch.int32, device=DEV),
                                qkv_dtype=dt, cu_seqlens_q=cq, causal=True)
    o1, l1 = flash_attn_varlen_func(q, k, v, cq, ck, max(lq), max(lk), causal=True, return_attn_probs=True,
                                    scheduler_metadata=md)
    o0, l0 = flash_attn_varlen_func(q, k, v, cq, ck, max(lq), max(lk), causal=True, num_splits=0,
                                    return_attn_probs=True)
    torch.cuda.synchronize()
    assert _same(o0, o1) and _same(l0, l1), "metadata changed the result"
    ro, rl = orc.attention(bits(q), bits(k), bits(v), dtype=odt(dt), scale=D ** -0.5, causal=True,
                           cu_seqlens_q=cq.cpu().numpy(), cu_seqlens_k=ck.cpu().numpy(), max_seqlen_q=max(lq),
                           nthreads=NT)
    assert_close_out(o1, ro, dt)
    assert_close_lse(l1, rl)
    with pytest.raises(RuntimeError, match="different call"):
        flash_attn_varlen_func(q, k, v, cq, ck, max(lq), max(lk), causal=False, scheduler_metadata=md)


def _paged(B, L, page, Hk, D, dt, g, extra=0):
    need = [(int(x) + extra + page - 1) // page for x in L]
    nb = sum(need) + 3
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt = torch.zeros((B, max(need)), dtype=torch.int32)
    o = 0
    for b in range(B):
        bt[b, :need[b]] = perm[o:o + need[b]]
        o += need[b]
    return bt, randn((nb, page, Hk, D), dt, g, "cpu"), randn((nb, page, Hk, D), dt, g, "cpu")


@pytest.mark.parametrize("sq", [1, 4])
def test_flash_attn_kvcache_metadata_bsnd(sq):
    from flash_attn_npu_v3 import flash_attn_with_kvcache, get_scheduler_metadata
    print(f"case metadata kvcache bsnd sq={sq}", flush=True)
    g = torch.Generator().manual_seed(702 + sq)
    B, H, Hk, D, page, dt = 5, 32, 8, 128, 64, torch.bfloat16
    L = np.array([700, 33, 4000, 1, 2500], np.int32)
    bt, kc, vc = _paged(B, L, page, Hk, D, dt, g, extra=sq)
    q = randn((B, sq, H, D), dt, g, "cpu")
    kn, vn = randn((B, sq, Hk, D), dt, g, "cpu"), randn((B, sq, Hk, D), dt, g, "cpu")
    sl = torch.from_numpy(L).to(DEV)
    md = get_scheduler_metadata(B, sq, bt.shape[1] * page, H, Hk, D, sl, qkv_dtype=dt, page_size=page, causal=True)
    res = []
    for use in (True, False):
        kcd, vcd = kc.to(DEV), vc.to(DEV)
        o, l, *_ = flash_attn_with_kvcache(q.to(DEV), kcd, vcd, k=kn.to(DEV), v=vn.to(DEV), cache_seqlens=sl,
                                           page_table=bt.to(DEV), causal=True, return_softmax_lse=True,
                                           scheduler_metadata=md if use else None)
        torch.cuda.synchronize()
        res.append((o, l, bits(kcd), bits(vcd)))
    (o1, l1, k1, v1), (o0, l0, k0, v0) = res
    assert _same(o0, o1) and _same(l0, l1) and np.array_equal(k0, k1) and np.array_equal(v0, v1)
    ro, rl, rk, _ = orc.kvcache_forward(bits(q), bits(kc), bits(vc), dtype=odt(dt), cache_seqlens=L, k=bits(kn),
                                        v=bits(vn), block_table=bt.numpy(), causal=True, nthreads=NT)
    assert np.array_equal(k1, rk), "append not bit-exact"
    assert_close_out(o1, ro, dt)
    assert_close_lse(l1, rl)
    with pytest.raises(RuntimeError, match="different call"):
        flash_attn_with_kvcache(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_seqlens=sl, page_table=bt.to(DEV),
                                causal=False, scheduler_metadata=md)
    # a copy of the metadata is checked through its header (reading it back)
    flash_attn_with_kvcache(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_seqlens=sl, page_table=bt.to(DEV), causal=True,
                            scheduler_metadata=md.clone())


def test_flash_attn_kvcache_metadata_tnd():
    from flash_attn_npu_v3 import flash_attn_with_kvcache, get_scheduler_metadata
    print("case metadata kvcache tnd", flush=True)
    g = torch.Generator().manual_seed(705)
    H, Hk, D, page, dt = 16, 4, 128, 128, torch.float16
    lq, L = [3, 1, 7], np.array([200, 64, 1000], np.int32)
    bt, kc, vc = _paged(3, L, page, Hk, D, dt, g)
    cq = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    q = randn((int(cq[-1]), H, D), dt, g, "cpu")
    sl = torch.from_numpy(L).to(DEV)
    cqd = torch.from_numpy(cq).to(DEV)
    md = get_scheduler_metadata(3, max(lq), bt.shape[1] * page, H, Hk, D, sl, qkv_dtype=dt, cu_seqlens_q=cqd,
                                page_size=page, causal=True)
    outs = []
    for use in (True, False):
        o, l, *_ = flash_attn_with_kvcache(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_seqlens=sl, page_table=bt.to(DEV),
                                           cu_seqlens_q=cqd, max_seqlen_q=max(lq), causal=True,
                                           return_softmax_lse=True, scheduler_metadata=md if use else None)
        outs.append((o, l))
    torch.cuda.synchronize()
    assert _same(outs[0][0], outs[1][0]) and _same(outs[0][1], outs[1][1])
    ro, rl = orc.attention(bits(q), bits(kc), bits(vc), dtype=odt(dt), scale=D ** -0.5, causal=True,
                           cu_seqlens_q=cq, max_seqlen_q=max(lq), seqlens_k=L, block_table=bt.numpy(), nthreads=NT)
    assert_close_out(outs[0][0], ro, dt)
    assert_close_lse(outs[0][1], rl)
    with pytest.raises(RuntimeError, match="different call"):
        flash_attn_with_kvcache(q.to(DEV), kc.to(DEV), vc.to(DEV), cache_seqlens=sl, page_table=bt.to(DEV),
                                causal=True, scheduler_metadata=md)  # dense q against TND metadata


@pytest.mark.parametrize("ns", [1, 3])
def test_kvcache_decode_forced_split_count(ns):
    """A forced num_splits on a decode-shaped call is honoured, as the
    reference's fixed split is (csrc/arch22/flash_attn_npu_v3/fa_split.h:335-402):
    the plan's per-sequence split count, read back from the metadata's
    workspace, is ns for every sequence (a 2-key sequence included, whose third
    chunk is empty), the append is bit-exact and the result is the oracle's."""
    from flash_attn_npu_v3 import flash_attn_with_kvcache, get_scheduler_metadata
    print(f"case kvcache decode forced num_splits={ns}", flush=True)
    g = torch.Generator().manual_seed(710 + ns)
    B, H, Hk, D, page, dt = 6, 64, 8, 128, 256, torch.bfloat16
    L = np.array([16, 300, 3000, 1, 2047, 900], np.int32)
    bt, kc, vc = _paged(B, L, page, Hk, D, dt, g, extra=1)
    q = randn((B, 1, H, D), dt, g, "cpu")
    kn, vn = randn((B, 1, Hk, D), dt, g, "cpu"), randn((B, 1, Hk, D), dt, g, "cpu")
    sl = torch.from_numpy(L).to(DEV)
    md = get_scheduler_metadata(B, 1, bt.shape[1] * page, H, Hk, D, sl, qkv_dtype=dt, page_size=page, causal=True,
                                num_splits=ns)
    kcd, vcd = kc.to(DEV), vc.to(DEV)
    o, l, *_ = flash_attn_with_kvcache(q.to(DEV), kcd, vcd, k=kn.to(DEV), v=vn.to(DEV), cache_seqlens=sl,
                                       page_table=bt.to(DEV), causal=True, return_softmax_lse=True, num_splits=ns,
                                       scheduler_metadata=md)
    torch.cuda.synchronize()
    # the workspace starts with the plan table: B + 1 item offsets, then the
    # split count of each sequence
    sched = md[256:256 + 4 * (2 * B + 2)].cpu().numpy().view(np.int32)
    assert (sched[B + 1:2 * B + 1] == ns).all(), sched
    ro, rl, rk, rv = orc.kvcache_forward(bits(q), bits(kc), bits(vc), dtype=odt(dt), cache_seqlens=L, k=bits(kn),
                                         v=bits(vn), block_table=bt.numpy(), causal=True, nthreads=NT)
    assert np.array_equal(bits(kcd), rk) and np.array_equal(bits(vcd), rv), "append not bit-exact"
    assert_close_out(o, ro, dt)
    assert_close_lse(l, rl)
