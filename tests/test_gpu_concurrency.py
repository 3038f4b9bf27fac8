"""Calls from several host threads at once, each on its own stream: the
library keeps no shared mutable state (plans are made per call, workspaces
come from the caller's stream, error messages are per thread), so every
concurrent result equals the same call made alone, bit for bit, and one
thread's validation errors never show up in another thread's message."""
import threading

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bits(t):
    t = t.detach()
    return t.view(torch.int32).cpu().numpy() if t.dtype == torch.float32 else t.view(torch.int16).cpu().numpy()


def _workloads():
    import flash_attn_npu_v2
    import flash_attn_npu_v3
    g = torch.Generator(device=DEV).manual_seed(90)
    r = lambda *s: torch.randn(s, generator=g, device=DEV, dtype=torch.float32).to(torch.bfloat16)
    B, H, Hk, D = 6, 32, 8, 128
    q1, kc1, vc1 = r(B, 1, H, D), r(B, 4096, Hk, D), r(B, 4096, Hk, D)
    sl1 = torch.tensor([100, 4000, 2500, 7, 3333, 1024], dtype=torch.int32, device=DEV)
    q2, k2, v2 = r(2, 700, H, D), r(2, 900, Hk, D), r(2, 900, Hk, D)
    q3, kc3, vc3 = r(2, 64, 16, 64), r(2, 2048, 4, 64), r(2, 2048, 4, 64)
    sl3 = torch.tensor([1500, 300], dtype=torch.int32, device=DEV)
    q4, k4, v4, do4 = r(1, 512, 8, 128), r(1, 512, 2, 128), r(1, 512, 2, 128), r(1, 512, 8, 128)

    def decode():
        o, l = flash_attn_npu_v2.flash_attn_with_kvcache(q1, kc1, vc1, cache_seqlens=sl1, causal=True,
                                                         return_softmax_lse=True)
        return [o, l]

    def dense():
        o, l, _ = flash_attn_npu_v2.flash_attn_func(q2, k2, v2, causal=True, return_attn_probs=True)
        return [o, l]

    def split_decode():
        o, l, *_ = flash_attn_npu_v3.flash_attn_with_kvcache(q3, kc3, vc3, cache_seqlens=sl3, causal=True,
                                                             num_splits=3, return_softmax_lse=True)
        return [o, l]

    def backward():
        qd, kd, vd = (x.clone().requires_grad_(True) for x in (q4, k4, v4))
        o = flash_attn_npu_v2.flash_attn_func(qd, kd, vd, causal=True)
        return list(torch.autograd.grad(o, (qd, kd, vd), do4))

    return [decode, dense, split_decode, backward]


def test_threads_on_separate_streams_match_serial_calls():
    print("case concurrency: 4 threads x 4 workloads x 8 repeats on 4 streams", flush=True)
    works = _workloads()
    ref = [[_bits(t) for t in w()] for w in works]
    torch.cuda.synchronize()
    errors = []

    def worker(tid):
        s = torch.cuda.Stream()
        try:
            with torch.cuda.stream(s):
                for rep in range(8):
                    w = (tid + rep) % len(works)
                    outs = works[w]()
                    s.synchronize()
                    for a, b in zip(outs, ref[w]):
                        if not np.array_equal(_bits(a), b):
                            errors.append(f"thread {tid} rep {rep} workload {w} differs")
        except Exception as e:  # noqa: BLE001  (reported below)
            errors.append(f"thread {tid}: {type(e).__name__}: {e}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    torch.cuda.synchronize()
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors[:4]


def test_error_messages_stay_in_their_thread():
    """The C ABI's last-error message is per thread: a thread whose calls are
    refused reads its own message while other threads run valid calls."""
    from fa_mi355x import capi
    print("case concurrency: per-thread error messages", flush=True)
    q = torch.zeros((1, 1, 4, 128), dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros((1, 64, 4, 128), dtype=torch.bfloat16, device=DEV)
    out, lse = torch.empty_like(q), torch.empty((1, 4, 1), dtype=torch.float32, device=DEV)
    sl = torch.tensor([10], dtype=torch.int32, device=DEV)
    P = lambda t: t.data_ptr()

    def params(headdim, nheads_k):
        return capi.new_params(dtype=capi.FA_DTYPE_BF16, batch=1, seqlen_q=1, nheads=4, nheads_k=nheads_k,
                               headdim=headdim, headdim_v=headdim, seqlen_k=64, batch_cache=1, q=P(q),
                               q_batch_stride=q.stride(0), q_row_stride=q.stride(1), q_head_stride=q.stride(2),
                               k=P(kc), k_batch_stride=kc.stride(0), k_row_stride=kc.stride(1),
                               k_head_stride=kc.stride(2), v=P(kc), v_batch_stride=kc.stride(0),
                               v_row_stride=kc.stride(1), v_head_stride=kc.stride(2), out=P(out),
                               out_batch_stride=out.stride(0), out_row_stride=out.stride(1),
                               out_head_stride=out.stride(2), softmax_lse=P(lse), cache_seqlens=P(sl),
                               softmax_scale=0.1, is_causal=1)
    bad = []

    def refusing(p, expect):
        def run():
            good = params(128, 4)
            for _ in range(300):
                st, _n = capi.workspace_size(p, capi.FA_KIND_KVCACHE)
                msg = capi.last_error()
                if st == capi.FA_OK or expect not in msg:
                    bad.append(f"expected {expect!r}, read {st}: {msg!r}")
                    return
                st, _n = capi.workspace_size(good, capi.FA_KIND_KVCACHE)  # a valid call in between
                if st != capi.FA_OK:
                    bad.append(f"valid call refused: {capi.last_error()!r}")
                    return
        return run

    # two kinds of refusal with different messages, two threads each
    kinds = [(params(512, 4), "head dimension"), (params(128, 3), "must divide")]
    threads = [threading.Thread(target=refusing(*kinds[i % 2])) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not bad, bad[:4]
