"""HIP-graph capture of the forward calls (the drop-in boundary promises that a
call is capturable once its shapes are fixed: no host synchronisation, no
device-to-host reads, no hipMemset, workspace from the caching allocator).

Each graph is replayed several times with eager work and synchronisations in
between, and every replay is compared bit for bit with the eager result of the
same call."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _randn(shape, dtype, g):
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype).to(DEV)


def _replay_and_check(fn, outs_eager, n=4):
    """Capture fn() and compare n replays with outs_eager."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm the caching allocator outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = fn()
    for rep in range(n):
        # unrelated eager work between replays
        junk = torch.randn(1 << 20, device=DEV)
        junk.mul_(2.0).add_(1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, outs_eager):
            assert torch.equal(o, e), f"replay {rep} differs from the eager result"


@pytest.mark.parametrize("num_splits", [0, 3])
def test_graph_decode_with_append(num_splits):
    """num_splits 0: the decode kernel (append fused) and its merge; 3: a
    forced split count, which runs the append kernel, the split prefill
    kernel and its merge."""
    import flash_attn_npu_v2
    print(f"case graph decode num_splits={num_splits}", flush=True)
    g = torch.Generator().manual_seed(70)
    B, H, Hk, D, cap = 8, 32, 8, 128, 2048
    q = _randn((B, 1, H, D), torch.bfloat16, g)
    kc = _randn((B, cap, Hk, D), torch.bfloat16, g)
    vc = _randn((B, cap, Hk, D), torch.bfloat16, g)
    kn = _randn((B, 1, Hk, D), torch.bfloat16, g)
    vn = _randn((B, 1, Hk, D), torch.bfloat16, g)
    seqlens = torch.randint(100, cap - 1, (B,), generator=g, dtype=torch.int32).to(DEV)

    def fn():
        return flash_attn_npu_v2.flash_attn_with_kvcache(q, kc, vc, k=kn, v=vn, cache_seqlens=seqlens, causal=True,
                                                         num_splits=num_splits, return_softmax_lse=True)

    eager = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    _replay_and_check(fn, eager)


def test_graph_chunked_prefill_rotary_paged():
    import flash_attn_npu_v2
    print("case graph chunked prefill rotary paged", flush=True)
    g = torch.Generator().manual_seed(71)
    B, Sq, H, Hk, D, page = 2, 96, 16, 4, 128, 64
    L = [300, 111]
    need = [(x + Sq + page - 1) // page for x in L]
    nb = sum(need) + 2
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt = torch.zeros((B, max(need)), dtype=torch.int32)
    o = 0
    for b in range(B):
        bt[b, :need[b]] = perm[o:o + need[b]]
        o += need[b]
    bt = bt.to(DEV)
    q = _randn((B, Sq, H, D), torch.bfloat16, g)
    kc = _randn((nb, page, Hk, D), torch.bfloat16, g)
    vc = _randn((nb, page, Hk, D), torch.bfloat16, g)
    kn = _randn((B, Sq, Hk, D), torch.bfloat16, g)
    vn = _randn((B, Sq, Hk, D), torch.bfloat16, g)
    inv = 1.0 / (10000 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    ang = torch.arange(1024, dtype=torch.float32)[:, None] * inv[None, :]
    cos, sin = torch.cos(ang).to(torch.bfloat16).to(DEV), torch.sin(ang).to(torch.bfloat16).to(DEV)
    seqlens = torch.tensor(L, dtype=torch.int32, device=DEV)

    def fn():
        return flash_attn_npu_v2.flash_attn_with_kvcache(q, kc, vc, k=kn, v=vn, rotary_cos=cos, rotary_sin=sin,
                                                         cache_seqlens=seqlens, block_table=bt, causal=True,
                                                         rotary_interleaved=False, return_softmax_lse=True)

    eager = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    _replay_and_check(fn, eager)


def test_graph_dense_split():
    import flash_attn_npu_v2
    print("case graph dense with split", flush=True)
    g = torch.Generator().manual_seed(72)
    # one sequence, few row tiles: the prefill kernel splits the key range and merges
    q = _randn((1, 200, 8, 128), torch.float16, g)
    k = _randn((1, 3000, 2, 128), torch.float16, g)
    v = _randn((1, 3000, 2, 128), torch.float16, g)

    def fn():
        out, lse, _ = flash_attn_npu_v2.flash_attn_func(q, k, v, causal=True, return_attn_probs=True)
        return out, lse

    eager = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    _replay_and_check(fn, eager)


def test_graph_v3_ragged_kvcache_leftpad_chunk():
    """The v3 operator with ragged queries and new tokens, cache_leftpad,
    rotary_seqlens and attention_chunk: a serving step captured once."""
    import flash_attn_npu_v3
    print("case graph v3 ragged kvcache", flush=True)
    g = torch.Generator().manual_seed(73)
    H, Hk, D, cap = 16, 4, 128, 1024
    q_lens, new_lens = [1, 40, 3], [1, 40, 3]
    cu_q = torch.tensor([0, 1, 41, 44], dtype=torch.int32, device=DEV)
    cu_n = torch.tensor([0, 1, 41, 44], dtype=torch.int32, device=DEV)
    q = _randn((sum(q_lens), H, D), torch.bfloat16, g)
    kn = _randn((sum(new_lens), Hk, D), torch.bfloat16, g)
    vn = _randn((sum(new_lens), Hk, D), torch.bfloat16, g)
    kc = _randn((3, cap, Hk, D), torch.bfloat16, g)
    vc = _randn((3, cap, Hk, D), torch.bfloat16, g)
    inv = 1.0 / (10000 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    ang = torch.arange(2048, dtype=torch.float32)[:, None] * inv[None, :]
    cos, sin = torch.cos(ang).to(torch.bfloat16).to(DEV), torch.sin(ang).to(torch.bfloat16).to(DEV)
    seqlens = torch.tensor([500, 0, 900], dtype=torch.int32, device=DEV)
    leftpad = torch.tensor([100, 0, 7], dtype=torch.int32, device=DEV)
    rot = torch.tensor([400, 0, 893], dtype=torch.int32, device=DEV)

    def fn():
        out, lse, *_ = flash_attn_npu_v3.flash_attn_with_kvcache(
            q, kc, vc, k=kn, v=vn, rotary_cos=cos, rotary_sin=sin, cache_seqlens=seqlens, cache_leftpad=leftpad,
            cu_seqlens_q=cu_q, cu_seqlens_k_new=cu_n, max_seqlen_q=40, rotary_seqlens=rot, causal=True,
            attention_chunk=256, rotary_interleaved=False, return_softmax_lse=True)
        return out, lse

    eager = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    _replay_and_check(fn, eager)


def test_graph_backward():
    """Forward and backward of flash_attn_func captured together (a training step)."""
    import flash_attn_npu_v2
    print("case graph backward", flush=True)
    g = torch.Generator().manual_seed(74)
    q = _randn((2, 300, 8, 128), torch.bfloat16, g).requires_grad_(True)
    k = _randn((2, 300, 2, 128), torch.bfloat16, g).requires_grad_(True)
    v = _randn((2, 300, 2, 128), torch.bfloat16, g).requires_grad_(True)
    do = _randn((2, 300, 8, 128), torch.bfloat16, g)

    def fn():
        out = flash_attn_npu_v2.flash_attn_func(q, k, v, causal=True)
        dq, dk, dv = torch.autograd.grad(out, (q, k, v), do)
        return out.detach(), dq, dk, dv

    eager = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    _replay_and_check(fn, eager)
