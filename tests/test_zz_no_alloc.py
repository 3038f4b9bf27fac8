"""fa_mha_fwd_kvcache_noalloc (the kvcache forward on the library's static
scratch, for callers that cannot allocate) against fa_mha_fwd_kvcache with a
caller workspace, both through the C ABI: two calls in a row, the second with
a smaller input, each compared bit for bit (out, LSE and the cache after the
append), and a call whose scratch need exceeds the limit is refused; the
calls leave device free memory unchanged and replay bitwise under HIP graph
capture."""
import ctypes

import numpy as np
import pytest
import torch

from tests._util import bits, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lib():
    from fa_mi355x import capi
    return capi, capi.lib()


def _decode_call(capi, B, H, Hk, D, cap, seqlens, seed, page=0, num_splits=0, Sq=1):
    """Tensors and fa_fwd_params of a bf16 GQA decode with a 1-token append
    (paged when page > 0); returns (params, tensors)."""
    g = torch.Generator().manual_seed(seed)
    dt = torch.bfloat16
    q = randn((B, Sq, H, D), dt, g, DEV)
    if page:
        need = [(int(L) + 1 + page - 1) // page for L in seqlens]
        nb = sum(need) + 4
        perm = torch.randperm(nb, generator=g).to(torch.int32)
        bt = torch.zeros((B, max(need)), dtype=torch.int32)
        o = 0
        for b in range(B):
            bt[b, :need[b]] = perm[o:o + need[b]]
            o += need[b]
        bt = bt.to(DEV)
        kc = randn((nb, page, Hk, D), dt, g, DEV)
        vc = randn((nb, page, Hk, D), dt, g, DEV)
    else:
        bt = None
        kc = randn((B, cap, Hk, D), dt, g, DEV)
        vc = randn((B, cap, Hk, D), dt, g, DEV)
    kn = randn((B, 1, Hk, D), dt, g, DEV)
    vn = randn((B, 1, Hk, D), dt, g, DEV)
    sl = torch.as_tensor(np.asarray(seqlens, np.int32)).to(DEV)
    out = torch.empty_like(q)
    lse = torch.empty((B, H, Sq), dtype=torch.float32, device=DEV)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    kw = dict(dtype=capi.FA_DTYPE_BF16, batch=B, seqlen_q=Sq, nheads=H, nheads_k=Hk, headdim=D, headdim_v=D,
              seqlen_k=kc.shape[1], batch_cache=kc.shape[0], q=P(q), q_batch_stride=q.stride(0),
              q_row_stride=q.stride(1), q_head_stride=q.stride(2), k=P(kc), k_batch_stride=kc.stride(0),
              k_row_stride=kc.stride(1), k_head_stride=kc.stride(2), v=P(vc), v_batch_stride=vc.stride(0),
              v_row_stride=vc.stride(1), v_head_stride=vc.stride(2), k_new=P(kn), knew_batch_stride=kn.stride(0),
              knew_row_stride=kn.stride(1), knew_head_stride=kn.stride(2), v_new=P(vn),
              vnew_batch_stride=vn.stride(0), vnew_row_stride=vn.stride(1), vnew_head_stride=vn.stride(2),
              seqlen_new=1, out=P(out), out_batch_stride=out.stride(0), out_row_stride=out.stride(1),
              out_head_stride=out.stride(2), softmax_lse=P(lse), cache_seqlens=P(sl), softmax_scale=D ** -0.5,
              is_causal=1, num_splits=num_splits)
    if bt is not None:
        kw.update(block_table=P(bt), block_table_batch_stride=bt.stride(0), max_blocks_per_seq=bt.shape[1],
                  block_table_rows=bt.shape[0], page_block_size=page)
    p = capi.new_params(**kw)
    return p, dict(q=q, kc=kc, vc=vc, kn=kn, vn=vn, sl=sl, out=out, lse=lse, bt=bt)


def _run_pair(capi, L, shape, page, seed, num_splits=0):
    """The same call twice on separate copies of the caches: with a workspace,
    then without; returns both results."""
    stream = torch.cuda.current_stream().cuda_stream
    res = []
    for noalloc in (False, True):
        p, t = _decode_call(capi, *shape, seed=seed, page=page, num_splits=num_splits)
        if noalloc:
            st = L.fa_mha_fwd_kvcache_noalloc(ctypes.byref(p), stream)
        else:
            st, n = capi.workspace_size(p, capi.FA_KIND_KVCACHE)
            assert st == capi.FA_OK, capi.last_error()
            ws = torch.empty(max(n, 256), dtype=torch.uint8, device=DEV)
            p.workspace, p.workspace_bytes = ctypes.c_void_p(ws.data_ptr()), ws.numel()
            st = capi.forward(p, capi.FA_KIND_KVCACHE, stream)
        assert st == capi.FA_OK, capi.last_error()
        torch.cuda.synchronize()
        res.append((bits(t["out"]), t["lse"].cpu().numpy().view(np.uint32), bits(t["kc"]), bits(t["vc"])))
    return res


def test_noalloc_matches_workspace_entry_point():
    capi, L = _lib()
    rng = np.random.default_rng(900)
    # first call: config-2-like decode whose segments are cut across many
    # wave workers (partials in the scratch); second: a smaller paged call;
    # third: a decode with a forced split count, which runs the split prefill
    # path (its sched table and partial rows in the scratch)
    shapes = [
        (24, 32, 8, 128, 8192, rng.integers(1024, 8191, 24), 0, 0),
        (5, 64, 8, 128, 0, rng.integers(10, 3000, 5), 64, 0),
        (4, 32, 8, 128, 4096, rng.integers(500, 4000, 4), 0, 3),
    ]
    for i, (B, H, Hk, D, cap, sl, page, ns) in enumerate(shapes):
        print(f"case noalloc call {i}: B{B} H{H}/{Hk} D{D} cap{cap} page{page} num_splits{ns}", flush=True)
        (o0, l0, k0, v0), (o1, l1, k1, v1) = _run_pair(capi, L, (B, H, Hk, D, cap, sl), page, seed=900 + i,
                                                       num_splits=ns)
        assert np.array_equal(k0, k1) and np.array_equal(v0, v1), "caches differ after the append"
        assert np.array_equal(o0, o1), f"out differs in {(o0 != o1).sum()} elements"
        assert np.array_equal(l0, l1), f"lse differs in {(l0 != l1).sum()} elements"


def test_noalloc_refuses_scratch_above_limit():
    capi, L = _lib()
    print("case noalloc refuses an oversized scratch", flush=True)
    # a short-q prefill split 64 ways: partials of 64 x 256 rows x 128 fp32 per
    # (batch, kv head) tile, far beyond the static scratch
    p, _ = _decode_call(capi, 8, 32, 8, 128, 4096, [4000] * 8, seed=950, num_splits=64, Sq=64)
    st, need = capi.workspace_size(p, capi.FA_KIND_KVCACHE)
    assert st == capi.FA_OK and need > capi.NOALLOC_SCRATCH_BYTES, need
    st = L.fa_mha_fwd_kvcache_noalloc(ctypes.byref(p), torch.cuda.current_stream().cuda_stream)
    assert st == capi.FA_EWORKSPACE, (st, capi.last_error())
    assert "more than the" in capi.last_error()


def test_noalloc_allocates_nothing_and_replays_under_graph_capture():
    """The use the entry point is for: calls that allocate nothing, also when
    captured into a HIP graph. Device free memory is unchanged by eager calls
    (after a first call has loaded the kernels' code), and each replay of the
    captured call, with eager work between replays, gives bitwise the eager
    result (out and LSE cleared before each replay, so a replay that wrote
    nothing would fail)."""
    capi, L = _lib()
    print("case noalloc: free memory around eager calls, graph capture and replays", flush=True)
    rng = np.random.default_rng(960)
    p, t = _decode_call(capi, 16, 32, 8, 128, 8192, rng.integers(1024, 8191, 16), seed=960)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        sh = side.cuda_stream
        assert L.fa_mha_fwd_kvcache_noalloc(ctypes.byref(p), sh) == capi.FA_OK, capi.last_error()
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        for _ in range(3):
            assert L.fa_mha_fwd_kvcache_noalloc(ctypes.byref(p), sh) == capi.FA_OK, capi.last_error()
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
    assert free1 == free0, f"device free memory changed by {free0 - free1} bytes over three calls"
    ref = (bits(t["out"]), t["lse"].cpu().numpy().view(np.uint32), bits(t["kc"]), bits(t["vc"]))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        st = L.fa_mha_fwd_kvcache_noalloc(ctypes.byref(p), torch.cuda.current_stream().cuda_stream)
    assert st == capi.FA_OK, capi.last_error()
    for rep in range(3):
        t["out"].zero_()
        t["lse"].zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = (bits(t["out"]), t["lse"].cpu().numpy().view(np.uint32), bits(t["kc"]), bits(t["vc"]))
        for name, a, b in zip(("out", "lse", "k_cache", "v_cache"), got, ref):
            assert np.array_equal(a, b), f"replay {rep}: {name} differs from the eager call"
