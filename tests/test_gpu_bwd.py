"""GPU parity of the backward pass: dq, dk, dv from torch.autograd through the
public flash_attn_func / flash_attn_varlen_func (v2 and v3) against the
float64 backward oracle (oracle/fa_bwd_oracle.py), fed with the inputs and the
forward's own LSE exactly as the reference tests feed their golden
(tests/test_flash_attn_npu_v2_bwd.py:76-138 in the reference). That forward
(out and LSE) is itself checked against the forward oracle first.

Bar, the reference's: |got - ref| <= 1e-2 + 1e-2 * |ref| elementwise
(RTOL_GOLDEN = ATOL_GOLDEN = 1e-2, test_flash_attn_npu_v2_bwd.py:27-28), on
inputs uniform in [-1, 1) (INPUT_LIMIT = 2, :31,63-64). Cases follow the
reference's lists (:146-330) at sizes the float64 oracle finishes quickly."""
import os

import numpy as np
import pytest
import torch

from oracle import fa_bwd_oracle as bo
from oracle import fa_oracle as orc
from tests._util import assert_close_lse, assert_close_out, bits, odt

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL = ATOL = 1e-2
NT = min(16, os.cpu_count() or 1)


def rand_inputs(shape, dtype, g):
    return (2.0 * (torch.rand(shape, generator=g) - 0.5)).to(dtype)


def check(name, got, ref):
    got = got.detach().float().cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    err = np.abs(got - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{name}: {int(bad.sum())} elements out of tolerance, max err {err.max():.3e}"


def check_forward(out, lse, q, k, v, dtype, scale, causal, window, softcap, alibi=None, chunk=0, cu_q=None,
                  cu_k=None):
    """The forward the gradients start from (out, and the LSE the backward
    recomputes P from) against the forward oracle, so an LSE error cannot
    cancel out in the gradient check."""
    ro, rl = orc.attention(bits(q), bits(k), bits(v), dtype=odt(dtype), scale=scale, softcap=softcap, causal=causal,
                           window=window, alibi=alibi, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                           max_seqlen_q=None if cu_q is None else int(np.diff(cu_q).max()), nthreads=NT, chunk=chunk)
    assert_close_out(out, ro, dtype)
    assert_close_lse(lse, rl)


def run_dense(dtype, B, H, Hk, Sq, Sk, D, causal, window=(-1, -1), softcap=0.0, alibi=False, api="v2", seed=0,
              chunk=0):
    import flash_attn_npu_v2
    import flash_attn_npu_v3
    print(f"case bwd dense {api} {dtype} B{B} H{H}/{Hk} {Sq}x{Sk} D{D} causal={causal} window={window} "
          f"softcap={softcap} alibi={alibi} chunk={chunk}", flush=True)
    g = torch.Generator().manual_seed(seed)
    q = rand_inputs((B, Sq, H, D), dtype, g)
    k = rand_inputs((B, Sk, Hk, D), dtype, g)
    v = rand_inputs((B, Sk, Hk, D), dtype, g)
    do = rand_inputs((B, Sq, H, D), dtype, g)
    slopes = torch.tensor([2.0 ** (-8.0 * (h + 1) / H) for h in range(H)], dtype=torch.float32) if alibi else None
    scale = D ** -0.5
    qd, kd, vd = (x.to(DEV).requires_grad_(True) for x in (q, k, v))
    if api == "v2":
        out, lse, _ = flash_attn_npu_v2.flash_attn_func(qd, kd, vd, causal=causal, window_size=window, softcap=softcap,
                                                        alibi_slopes=None if slopes is None else slopes.to(DEV),
                                                        return_attn_probs=True)
    else:
        out, lse = flash_attn_npu_v3.flash_attn_func(qd, kd, vd, causal=causal, window_size=window, softcap=softcap,
                                                     attention_chunk=chunk, return_attn_probs=True)
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), do.to(DEV))
    torch.cuda.synchronize()
    check_forward(out, lse, q, k, v, dtype, scale, causal, window, softcap,
                  alibi=None if slopes is None else slopes.numpy(), chunk=chunk)
    rq, rk, rv = bo.attention_bwd(q.float().numpy(), k.float().numpy(), v.float().numpy(), do.float().numpy(),
                                  lse.detach().cpu().numpy(), scale=scale, softcap=softcap, causal=causal,
                                  window=window, alibi=None if slopes is None else slopes.numpy(), chunk=chunk)
    check("dq", dq, rq)
    check("dk", dk, rk)
    check("dv", dv, rv)


def run_varlen(dtype, H, Hk, lq, lk, D, causal, window=(-1, -1), softcap=0.0, api="v2", seed=0, chunk=0):
    import flash_attn_npu_v2
    import flash_attn_npu_v3
    print(f"case bwd varlen {api} {dtype} H{H}/{Hk} lq={lq} lk={lk} D{D} causal={causal} window={window} "
          f"softcap={softcap}", flush=True)
    g = torch.Generator().manual_seed(seed)
    cq = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    ck = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
    q = rand_inputs((int(cq[-1]), H, D), dtype, g)
    k = rand_inputs((int(ck[-1]), Hk, D), dtype, g)
    v = rand_inputs((int(ck[-1]), Hk, D), dtype, g)
    do = rand_inputs((int(cq[-1]), H, D), dtype, g)
    scale = D ** -0.5
    qd, kd, vd = (x.to(DEV).requires_grad_(True) for x in (q, k, v))
    cqd, ckd = torch.from_numpy(cq).to(DEV), torch.from_numpy(ck).to(DEV)
    f = flash_attn_npu_v2.flash_attn_varlen_func if api == "v2" else flash_attn_npu_v3.flash_attn_varlen_func
    kw = dict(attention_chunk=chunk) if chunk else {}
    res = f(qd, kd, vd, cqd, ckd, max(lq), max(lk), causal=causal, window_size=window, softcap=softcap,
            return_attn_probs=True, **kw)
    out, lse = res[0], res[1]
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), do.to(DEV))
    torch.cuda.synchronize()
    check_forward(out, lse, q, k, v, dtype, scale, causal, window, softcap, chunk=chunk, cu_q=cq, cu_k=ck)
    rq, rk, rv = bo.attention_bwd(q.float().numpy(), k.float().numpy(), v.float().numpy(), do.float().numpy(),
                                  lse.detach().cpu().numpy(), scale=scale, softcap=softcap, causal=causal,
                                  window=window, cu_seqlens_q=cq, cu_seqlens_k=ck, chunk=chunk)
    check("dq", dq, rq)
    check("dk", dk, rk)
    check("dv", dv, rv)


# reference test_cases_bsnd (:146-163), sequence lengths halved
BSND = [
    (torch.float16, 1, 1, 1, 512, 512, 128, False, 0.0),
    (torch.float16, 3, 4, 4, 512, 512, 128, True, 0.0),
    (torch.float16, 4, 2, 1, 513, 513, 128, False, 0.0),
    (torch.bfloat16, 1, 1, 1, 512, 512, 128, False, 0.0),
    (torch.bfloat16, 3, 4, 4, 512, 512, 128, True, 0.0),
    (torch.bfloat16, 4, 2, 1, 513, 513, 128, False, 0.0),
    (torch.float16, 3, 4, 4, 512, 512, 128, True, 30.0),
    (torch.bfloat16, 4, 2, 1, 513, 513, 128, False, 30.0),
]


@pytest.mark.parametrize("case", BSND, ids=[f"bsnd{i}" for i in range(len(BSND))])
def test_bwd_dense(case):
    dtype, B, H, Hk, Sq, Sk, D, causal, softcap = case
    run_dense(dtype, B, H, Hk, Sq, Sk, D, causal, softcap=softcap, seed=sum(x for x in case if isinstance(x, int)))


# reference test_cases_bsnd_swa (:166-183)
SWA = [
    (torch.bfloat16, 1, 1, 1, 512, 512, 128, True, 256, 0, 0.0),
    (torch.bfloat16, 1, 1, 1, 512, 512, 128, True, 256, 128, 0.0),
    (torch.bfloat16, 3, 4, 4, 512, 512, 128, True, -128, 432, 0.0),
    (torch.bfloat16, 1, 1, 1, 512, 512, 128, False, 0, 128, 0.0),
    (torch.float16, 2, 2, 2, 512, 512, 128, False, 64, 128, 0.0),
    (torch.bfloat16, 1, 1, 1, 1, 1024, 128, True, 512, 0, 0.0),
    (torch.bfloat16, 2, 6, 2, 2, 1024, 128, True, -1, -1, 0.0),
    (torch.bfloat16, 2, 6, 2, 2, 1024, 128, True, 256, 0, 30.0),
    (torch.float16, 2, 2, 2, 512, 512, 128, False, 64, 128, 30.0),
]


@pytest.mark.parametrize("case", SWA, ids=[f"swa{i}" for i in range(len(SWA))])
def test_bwd_dense_window(case):
    dtype, B, H, Hk, Sq, Sk, D, causal, wl, wr, softcap = case
    run_dense(dtype, B, H, Hk, Sq, Sk, D, causal, window=(wl, wr), softcap=softcap, seed=sum(x for x in case if isinstance(x, int)))


# reference test_cases_varlen (:222-235): one sequence each, head dims 64 / 111 / 128
VARLEN = [
    (torch.bfloat16, 1, 1, [512], [1024], 128, True, 0.0),
    (torch.float16, 5, 1, [512], [512], 128, True, 0.0),
    (torch.bfloat16, 1, 1, [1777], [2048], 64, True, 0.0),
    (torch.bfloat16, 5, 1, [711], [2048], 111, True, 0.0),
    (torch.float16, 5, 1, [512], [512], 128, True, 30.0),
    (torch.bfloat16, 4, 2, [37, 1, 300, 128, 0], [37, 90, 300, 1000, 5], 128, True, 0.0),   # ragged, empty q
    (torch.float16, 4, 2, [100, 257], [80, 300], 64, False, 0.0),
]


@pytest.mark.parametrize("case", VARLEN, ids=[f"varlen{i}" for i in range(len(VARLEN))])
def test_bwd_varlen(case):
    dtype, H, Hk, lq, lk, D, causal, softcap = case
    run_varlen(dtype, H, Hk, lq, lk, D, causal, softcap=softcap, seed=len(lq) * 7 + D)


# reference test_cases_varlen_swa (:275-282)
VARLEN_SWA = [
    (torch.bfloat16, 1, 1, [512], [1024], 128, True, 512, 0, 0.0),
    (torch.bfloat16, 1, 1, [512], [1024], 128, False, 0, 256, 0.0),
    (torch.float16, 2, 2, [512], [512], 128, False, 64, 128, 0.0),
    (torch.bfloat16, 1, 1, [512], [1024], 128, False, 0, 256, 30.0),
]


@pytest.mark.parametrize("case", VARLEN_SWA, ids=[f"vswa{i}" for i in range(len(VARLEN_SWA))])
def test_bwd_varlen_window(case):
    dtype, H, Hk, lq, lk, D, causal, wl, wr, softcap = case
    run_varlen(dtype, H, Hk, lq, lk, D, causal, window=(wl, wr), softcap=softcap, seed=wl + 3 * wr + D)


# head dims above 128 (reference test_cases_varlen :225-226,231-232 use 192 and 256)
@pytest.mark.parametrize("case", [
    (torch.float16, 5, 1, [777], [888], 192, False, 0.0),
    (torch.float16, 5, 1, [777], [1000], 256, True, 0.0),
    (torch.float16, 5, 1, [777], [888], 192, False, 30.0),
    (torch.bfloat16, 4, 2, [300, 1, 129], [300, 64, 500], 256, True, 30.0),
], ids=["d192", "d256", "d192_softcap", "d256_ragged_softcap"])
def test_bwd_varlen_large_headdim(case):
    dtype, H, Hk, lq, lk, D, causal, softcap = case
    run_varlen(dtype, H, Hk, lq, lk, D, causal, softcap=softcap, seed=D + len(lq))


def test_bwd_dense_headdim_256_window_gqa():
    run_dense(torch.bfloat16, 2, 8, 2, 300, 333, 256, True, window=(100, 0), seed=17)


def test_bwd_dense_headdim_136():
    run_dense(torch.float16, 2, 4, 4, 200, 200, 136, False, seed=18)


def test_bwd_alibi():
    # ALiBi gradients (the reference's backward ignores alibi_slopes; here the
    # bias enters as in the forward)
    run_dense(torch.bfloat16, 2, 4, 2, 200, 300, 128, True, alibi=True, seed=11)


def test_bwd_headdim_64_gqa_causal():
    run_dense(torch.float16, 2, 8, 2, 300, 300, 64, True, seed=12)


# head dims up to 64 run the 64 backward kernels (32 keys per dK/dV wave, 32 rows per dQ wave)
@pytest.mark.parametrize("D", [32, 48, 64])
def test_bwd_headdim64_noncausal(D):
    run_dense(torch.bfloat16, 2, 4, 4, 333, 270, D, False, seed=20 + D)


def test_bwd_headdim64_window_softcap_alibi():
    run_dense(torch.bfloat16, 2, 8, 4, 400, 512, 64, True, window=(120, 0), softcap=25.0, alibi=True, seed=21)


def test_bwd_headdim64_varlen():
    run_varlen(torch.float16, 8, 2, [129, 1, 500, 64], [200, 33, 500, 64], 64, True, seed=22)


def test_bwd_v3_api():
    run_dense(torch.bfloat16, 2, 4, 2, 256, 384, 128, True, api="v3", seed=13)
    run_varlen(torch.bfloat16, 4, 2, [50, 200], [60, 260], 128, True, api="v3", seed=14)


def test_bwd_deterministic():
    """Two identical backward calls give bit-identical gradients (no atomics)."""
    import flash_attn_npu_v2
    print("case bwd deterministic", flush=True)
    g = torch.Generator().manual_seed(15)
    q, k, v, do = (rand_inputs((2, 400, 8, 128), torch.bfloat16, g).to(DEV) for _ in range(4))
    k, v = k[:, :, :2].contiguous(), v[:, :, :2].contiguous()
    res = []
    for _ in range(2):
        qd, kd, vd = (x.clone().requires_grad_(True) for x in (q, k, v))
        out = flash_attn_npu_v2.flash_attn_func(qd, kd, vd, causal=True)
        res.append(torch.autograd.grad(out, (qd, kd, vd), do))
    torch.cuda.synchronize()
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_bwd_softmax_d_returned():
    """_flash_attn_backward returns softmax_d = rowsum(dout * out) like the reference op."""
    from flash_attn_npu_v2.interface import _flash_attn_backward, _flash_attn_forward
    print("case bwd softmax_d", flush=True)
    g = torch.Generator().manual_seed(16)
    q, k, v, do = (rand_inputs((2, 100, 4, 128), torch.float16, g).to(DEV) for _ in range(4))
    out, lse, _, _ = _flash_attn_forward(q, k, v, 0.0, 128 ** -0.5, True)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    sd = _flash_attn_backward(do, q, k, v, out, lse, dq, dk, dv, 0.0, 128 ** -0.5, True, -1, 0, 0.0, None, False)
    torch.cuda.synchronize()
    ref = bo.softmax_d(out.float().cpu().numpy(), do.float().cpu().numpy())
    np.testing.assert_allclose(sd.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)


# attention_chunk (v3 API): the chunk cuts the causal / local band
@pytest.mark.parametrize("case", [
    (torch.bfloat16, 2, 4, 2, 512, 512, 128, True, (-1, -1), 64),
    (torch.float16, 1, 4, 4, 300, 700, 128, False, (-1, -1), 100),
    (torch.bfloat16, 2, 4, 1, 384, 384, 64, True, (90, 0), 128),
    (torch.bfloat16, 1, 4, 2, 200, 456, 256, True, (-1, -1), 48),
], ids=["causal64", "noncausal100", "window_d64", "d256"])
def test_bwd_chunk(case):
    dtype, B, H, Hk, Sq, Sk, D, causal, window, chunk = case
    run_dense(dtype, B, H, Hk, Sq, Sk, D, causal, window=window, api="v3", seed=B + H + Sq, chunk=chunk)


def test_bwd_varlen_chunk():
    run_varlen(torch.bfloat16, 4, 2, [130, 1, 260, 77], [130, 40, 300, 77], 128, True, api="v3", seed=9, chunk=96)


@pytest.mark.parametrize("D", [111, 36])
def test_bwd_v3_unaligned_headdim(D):
    # the v3 API runs head dims that are not a multiple of 8 zero-padded; the
    # gradients flow back through the padding
    run_dense(torch.bfloat16, 2, 4, 2, 200, 260, D, True, api="v3", seed=30 + D)


# GQA ratios that do not divide the dK/dV kernel's 64-row tiles: its per-thread
# row cursors move 64 packed rows per tile as 64 // g positions and 64 % g heads
# and carry a position when the head offset wraps; enough row tiles per key
# block that the wraps accumulate, and a left-only window for the reversed
# key-block order
@pytest.mark.parametrize("g", [3, 5, 7])
def test_bwd_gqa_ratio_not_dividing_row_tile(g):
    run_dense(torch.bfloat16, 1, 2 * g, 2, 700, 700, 128, True, seed=60 + g)
    run_dense(torch.float16, 2, g, 1, 333, 517, 64, False, window=(100, -1), seed=70 + g)
    run_varlen(torch.bfloat16, 2 * g, 2, [700, 1, 129], [700, 64, 300], 128, True, seed=80 + g)
