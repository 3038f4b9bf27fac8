"""GPU parity over a seeded random sweep of kvcache and dense calls: shapes,
head dims, GQA ratios, paging (page sizes on and off the fast path),
cache_batch_idx, appends with and without rotary, causal / local windows,
soft capping, ALiBi, forced split counts, both 16-bit dtypes and both APIs,
each against the CPU oracle at the north-star bar (run_kvcache / run_dense).
The list is drawn once from a fixed seed, so every run checks the same cases."""
import numpy as np
import pytest

from tests.test_gpu_parity import run_dense, run_kvcache

pytestmark = pytest.mark.gpu

HEADS = [(4, 4), (8, 2), (16, 4), (32, 8), (12, 3), (6, 1)]
DIMS = [64, 80, 96, 128, 128, 128, 192, 256]
SQS = [1, 1, 1, 2, 3, 4, 5, 8, 16, 33, 100, 257]
PAGES = [0, 0, 0, 16, 32, 64, 128, 256]


def _kv_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        H, Hk = HEADS[rng.integers(len(HEADS))]
        D = int(DIMS[rng.integers(len(DIMS))])
        Sq = int(SQS[rng.integers(len(SQS))])
        B = int(rng.integers(1, 9))
        page = int(PAGES[rng.integers(len(PAGES))])
        s_new = int(rng.choice([0, 0, 1, Sq]))
        seqlens = [int(x) for x in rng.integers(0, int(rng.choice([600, 3000, 9000])), B)]
        rotary = None
        if s_new and rng.random() < 0.4:
            # a rotary dim must be a multiple of 16 (as in Dao's kvcache rotary);
            # "partial" rotates the first D / 2 dims
            rotary = str(rng.choice(["neox", "interleaved", "partial"]))
            if rotary == "partial" and (D // 2) % 16:
                rotary = "neox"
        causal = bool(rng.random() < 0.7)
        window = (-1, -1)
        r = rng.random()
        if r < 0.25:
            window = (int(rng.integers(0, 2000)), 0 if causal else int(rng.integers(0, 50)))
        elif r < 0.35 and not causal:
            window = (-1, int(rng.integers(0, 100)))
        api = "v3" if rng.random() < 0.35 else "v2"
        alibi = api == "v2" and rng.random() < 0.3
        softcap = float(rng.choice([0.0, 0.0, 0.0, 30.0]))
        batch_idx = bool(rng.random() < 0.25)
        num_splits = int(rng.choice([0, 0, 0, 1, 3]))
        dtype = str(rng.choice(["bf16", "fp16"]))
        capacity = max(seqlens) + s_new + int(rng.integers(0, 64)) if not page else 0
        cases.append(dict(B=B, Sq=Sq, H=H, Hk=Hk, D=D, dtype=dtype, capacity=capacity, seqlens=seqlens, s_new=s_new,
                          page=page, rotary=rotary, causal=causal, window=window, alibi=alibi, batch_idx=batch_idx,
                          num_splits=num_splits, softcap=softcap, seed=1000 + i, api=api))
    return cases


def _dense_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        H, Hk = HEADS[rng.integers(len(HEADS))]
        D = int(DIMS[rng.integers(len(DIMS))])
        B = int(rng.integers(1, 4))
        Sq = int(rng.integers(1, 700))
        Sk = int(rng.integers(1, 900))
        causal = bool(rng.random() < 0.6)
        window = (-1, -1)
        if rng.random() < 0.3:
            window = (int(rng.integers(0, 500)), 0 if causal else int(rng.integers(0, 200)))
        cases.append(dict(B=B, Sq=Sq, Sk=Sk, H=H, Hk=Hk, D=D, dtype=str(rng.choice(["bf16", "fp16"])), causal=causal,
                          window=window, softcap=float(rng.choice([0.0, 0.0, 20.0])),
                          alibi=bool(rng.random() < 0.3), seed=2000 + i))
    return cases


KV_CASES = _kv_cases(200, 20251202)
DENSE_CASES = _dense_cases(48, 20251203)


def _dt(name):
    import torch
    return torch.bfloat16 if name == "bf16" else torch.float16


@pytest.mark.parametrize("i", range(len(KV_CASES)))
def test_random_kvcache(i):
    c = dict(KV_CASES[i])
    print(f"case random kvcache {i}: {c}", flush=True)
    c["dtype"] = _dt(c["dtype"])
    run_kvcache(**c)


@pytest.mark.parametrize("i", range(len(DENSE_CASES)))
def test_random_dense(i):
    c = dict(DENSE_CASES[i])
    print(f"case random dense {i}: {c}", flush=True)
    c["dtype"] = _dt(c["dtype"])
    run_dense(**c)


# ---- v3 kvcache extensions: ragged q and new tokens, cache_leftpad, any page size,
# rotary_seqlens, attention_chunk (run_v3 checks the caches bit for bit and the
# output / LSE against the v3 oracle) --------------------------------------------------------------

def _v3_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        H, Hk = HEADS[rng.integers(len(HEADS))]
        D = int(rng.choice([64, 96, 128, 128, 256, 111, 36]))
        B = int(rng.integers(1, 6))
        decode = rng.random() < 0.5
        q_lens = [int(x) for x in rng.integers(1, 5 if decode else 150, B)]
        ragged_q = bool(rng.random() < 0.5)
        if not ragged_q:
            q_lens = [q_lens[0]] * B
        ragged_new = bool(rng.random() < 0.4)
        if ragged_new:
            new_lens = [int(x) for x in rng.integers(0, 1 + max(q_lens), B)]
        else:
            new_lens = [int(rng.choice([0, 1, q_lens[0]]))] * B
        seqlens = [int(x) for x in rng.integers(0, int(rng.choice([300, 2000, 6000])), B)]
        page = int(rng.choice([0, 0, 1, 7, 16, 48, 64, 100, 256]))
        leftpad = None
        capacity = 0
        if page == 0:
            capacity = max(L + n for L, n in zip(seqlens, new_lens)) + 300
            if rng.random() < 0.4:
                leftpad = [int(x) for x in rng.integers(0, 300, B)]
        rotary = rot_dim = rotary_seqlens = None
        if max(new_lens) > 0 and rng.random() < 0.4:
            rotary = str(rng.choice(["neox", "interleaved"]))
            rot_dim = {111: 96, 36: 32}.get(D, D)
            if rng.random() < 0.4:
                rotary_seqlens = [int(x) for x in rng.integers(0, 500, B)]
        causal = bool(rng.random() < 0.7)
        window = (-1, -1)
        chunk = 0
        r = rng.random()
        if r < 0.2:
            window = (int(rng.integers(0, 1000)), 0 if causal else int(rng.integers(0, 40)))
        elif r < 0.35:
            chunk = int(rng.choice([32, 64, 100, 512]))
        cases.append(dict(H=H, Hk=Hk, D=D, dtype=str(rng.choice(["bf16", "fp16"])), q_lens=q_lens, new_lens=new_lens,
                          seqlens=seqlens, capacity=capacity, page=page, ragged_q=ragged_q, ragged_new=ragged_new,
                          leftpad=leftpad, rotary=rotary, rot_dim=rot_dim, rotary_seqlens=rotary_seqlens,
                          causal=causal, window=window, chunk=chunk, num_splits=int(rng.choice([0, 0, 1, 3])),
                          seed=3000 + i))
    return cases


V3_CASES = _v3_cases(120, 20251204)


@pytest.mark.parametrize("i", range(len(V3_CASES)))
def test_random_v3_kvcache(i):
    from tests.test_gpu_v3kv import run_v3
    c = dict(V3_CASES[i])
    print(f"case random v3 kvcache {i}: {c}", flush=True)
    c["dtype"] = _dt(c["dtype"])
    run_v3(**c)


# ---- backward: dense and varlen gradients against the fp64 oracle, the forward
# (out and LSE) against the forward oracle (run_dense / run_varlen of the
# backward tests) ----------------------------------------------------------------------------------

def _bwd_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        H, Hk = [(4, 4), (8, 2), (6, 1), (4, 1), (8, 8)][rng.integers(5)]
        D = int(rng.choice([40, 64, 80, 96, 128, 128, 192, 256]))
        api = "v3" if rng.random() < 0.35 else "v2"
        causal = bool(rng.random() < 0.6)
        window = (-1, -1)
        chunk = 0
        r = rng.random()
        if r < 0.25:
            window = (int(rng.integers(0, 300)), 0 if causal else int(rng.integers(0, 100)))
        elif r < 0.4 and api == "v3":
            chunk = int(rng.choice([32, 64, 100]))
        softcap = float(rng.choice([0.0, 0.0, 30.0]))
        alibi = api == "v2" and rng.random() < 0.25
        dtype = str(rng.choice(["bf16", "fp16"]))
        if rng.random() < 0.3:
            B = int(rng.integers(1, 4))
            lq = [int(x) for x in rng.integers(1, 300, B)]
            lk = [int(x) for x in rng.integers(1, 300, B)]
            cases.append(("varlen", dict(dtype=dtype, H=H, Hk=Hk, lq=lq, lk=lk, D=D, causal=causal, window=window,
                                         softcap=softcap, api=api, seed=4000 + i, chunk=chunk)))
        else:
            cases.append(("dense", dict(dtype=dtype, B=int(rng.integers(1, 3)), H=H, Hk=Hk,
                                        Sq=int(rng.integers(1, 400)), Sk=int(rng.integers(1, 400)), D=D,
                                        causal=causal, window=window, softcap=softcap, alibi=alibi, api=api,
                                        seed=4000 + i, chunk=chunk)))
    return cases


BWD_CASES = _bwd_cases(60, 20251205)


@pytest.mark.parametrize("i", range(len(BWD_CASES)))
def test_random_backward(i):
    from tests import test_gpu_bwd as tb
    kind, c = BWD_CASES[i]
    c = dict(c)
    print(f"case random backward {i}: {kind} {c}", flush=True)
    c["dtype"] = _dt(c["dtype"])
    (tb.run_varlen if kind == "varlen" else tb.run_dense)(**c)


# ---- FP8 (e4m3) forward: kvcache (contiguous or paged, decode- and prefill-shaped,
# forced split counts) and dense calls with or without descales, against the FP8
# oracle (exact widening, descaled scale, output times v_descale) ------------------------------------

def _fp8_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        H, Hk = HEADS[rng.integers(len(HEADS))]
        D = int(rng.choice([64, 96, 128, 128, 256]))
        causal = bool(rng.random() < 0.7)
        window = (-1, -1)
        if rng.random() < 0.25:
            window = (int(rng.integers(0, 800)), 0 if causal else int(rng.integers(0, 40)))
        common = dict(H=H, Hk=Hk, D=D, causal=causal, window=window, softcap=float(rng.choice([0.0, 0.0, 30.0])),
                      descale=bool(rng.random() < 0.8), seed=5000 + i)
        if rng.random() < 0.7:
            B = int(rng.integers(1, 6))
            cases.append(("kvcache", dict(common, B=B, Sq=int(rng.choice([1, 1, 2, 4, 16, 100])),
                                          L=[int(x) for x in rng.integers(1, int(rng.choice([500, 4000])), B)],
                                          page=int(rng.choice([0, 0, 16, 48, 64, 256])),
                                          num_splits=int(rng.choice([0, 0, 1, 3])))))
        else:
            cases.append(("dense", dict(common, B=int(rng.integers(1, 3)), Sq=int(rng.integers(1, 500)),
                                        Sk=int(rng.integers(1, 700)))))
    return cases


FP8_CASES = _fp8_cases(60, 20251206)


def _run_fp8(kind, B, H, Hk, D, causal, window, softcap, descale, seed, Sq, L=None, page=0, num_splits=0, Sk=0):
    import torch
    import flash_attn_npu_v3 as fa3
    from oracle import fa_oracle as orc
    from tests import test_gpu_fp8 as t8
    g = torch.Generator().manual_seed(seed)
    q = t8.fp8((B, Sq, H, D), g)
    qd = kd = vd = None
    if kind == "dense":
        k, v = t8.fp8((B, Sk, Hk, D), g), t8.fp8((B, Sk, Hk, D), g)
        if descale:
            qd, kd, vd = t8.descales(B, Hk, g)
        d = lambda x: None if x is None else x.to(t8.DEV)
        out, lse = fa3.flash_attn_func(q.to(t8.DEV), k.to(t8.DEV), v.to(t8.DEV), causal=causal, window_size=window,
                                       softcap=softcap, q_descale=d(qd), k_descale=d(kd), v_descale=d(vd),
                                       return_attn_probs=True)
        kx, vx, sk = t8.u8(k), t8.u8(v), None
    else:
        Lt = torch.tensor(L, dtype=torch.int32)
        if page:
            need = [(int(l) + page - 1) // page for l in L]
            mb = max(need)
            nblocks = sum(need) + 2
            perm = torch.randperm(nblocks, generator=g)
            bt = torch.zeros((B, mb), dtype=torch.int32)
            o = 0
            for b in range(B):
                bt[b, :need[b]] = perm[o:o + need[b]]
                o += need[b]
            kc, vc = t8.fp8((nblocks, page, Hk, D), g), t8.fp8((nblocks, page, Hk, D), g)
        else:
            bt = None
            cap = max(L) + 8
            kc, vc = t8.fp8((B, cap, Hk, D), g), t8.fp8((B, cap, Hk, D), g)
        if descale:
            qd, kd, vd = t8.descales(B, Hk, g)
        d = lambda x: None if x is None else x.to(t8.DEV)
        out, lse, *_ = fa3.flash_attn_with_kvcache(q.to(t8.DEV), kc.to(t8.DEV), vc.to(t8.DEV), cache_seqlens=d(Lt),
                                                   page_table=d(bt), q_descale=d(qd), k_descale=d(kd),
                                                   v_descale=d(vd), causal=causal, window_size=window,
                                                   softcap=softcap, num_splits=num_splits, return_softmax_lse=True)
        if page:
            kx = t8.u8(kc)[bt.numpy()].reshape(B, mb * page, Hk, D)
            vx = t8.u8(vc)[bt.numpy()].reshape(B, mb * page, Hk, D)
        else:
            kx, vx = t8.u8(kc), t8.u8(vc)
        sk = Lt.numpy()
    torch.cuda.synchronize()
    n = lambda x: None if x is None else x.numpy()
    ro, rl = orc.attention_fp8(t8.u8(q), kx, vx, scale=D ** -0.5, q_descale=n(qd), k_descale=n(kd),
                               v_descale=n(vd), causal=causal, window=window, softcap=softcap, seqlens_k=sk,
                               nthreads=t8.NT)
    t8.check(out, lse, ro, rl, vmax=1.0 if vd is None else float(vd.max()))


@pytest.mark.parametrize("i", range(len(FP8_CASES)))
def test_random_fp8(i):
    kind, c = FP8_CASES[i]
    print(f"case random fp8 {i}: {kind} {c}", flush=True)
    _run_fp8(kind, **c)


# ---- qv (scores add qv . v; decode-shaped kvcache calls, at most 16 packed rows
# per kv head) and pack_gqa=False, against the v3 oracle ----------------------------------------------

def _qv_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        H, Hk = HEADS[rng.integers(len(HEADS))]
        g = H // Hk
        D = int(rng.choice([64, 96, 128, 128]))
        B = int(rng.integers(1, 6))
        with_qv = bool(rng.random() < 0.6)
        smax = max(1, 16 // g) if with_qv else 40
        ragged = None
        Sq = int(rng.integers(1, smax + 1))
        if rng.random() < 0.3:
            ragged = [int(x) for x in rng.integers(1, smax + 1, B)]
        L = [int(x) for x in rng.integers(0, int(rng.choice([500, 3000])), B)]
        page = int(rng.choice([0, 0, 16, 64, 256]))
        new = int(rng.choice([0, 0, 1])) if ragged is None else 0
        capacity = 0 if page else max(L) + new + 16
        window = (-1, -1)
        if rng.random() < 0.25:
            window = (int(rng.integers(0, 600)), 0)
        cases.append(dict(B=B, Sq=Sq, H=H, Hk=Hk, D=D, dtype=str(rng.choice(["bf16", "fp16"])), L=L,
                          capacity=capacity, page=page, new=new, window=window, ragged=ragged,
                          pack_gqa=None if with_qv and rng.random() < 0.5 else False, seed=6000 + i,
                          with_qv=with_qv, softcap=float(rng.choice([0.0, 0.0, 5.0]))))
    return cases


QV_CASES = _qv_cases(48, 20251207)


@pytest.mark.parametrize("i", range(len(QV_CASES)))
def test_random_qv_pack_gqa(i):
    from tests.test_gpu_qv_packgqa import _kvcache_case
    c = dict(QV_CASES[i])
    print(f"case random qv / pack_gqa {i}: {c}", flush=True)
    c["dtype"] = _dt(c["dtype"])
    _kvcache_case(**c)


# ---- scheduler_metadata: a kvcache call given get_scheduler_metadata's plan
# (made for max_seqlen_q, the call may be shorter) gives bit for bit the result
# of the same call without it: the plan and workspace it carries cover the call ----------------------

def _md_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        H, Hk = HEADS[rng.integers(len(HEADS))]
        maxq = int(rng.choice([1, 2, 4, 8, 16, 64, 200]))
        causal = bool(rng.random() < 0.7)
        window = (-1, -1)
        if rng.random() < 0.25:
            window = (int(rng.integers(0, 1000)), 0 if causal else int(rng.integers(0, 40)))
        B = int(rng.integers(1, 9))
        cases.append(dict(B=B, H=H, Hk=Hk, D=int(rng.choice([64, 128, 128, 256])), maxq=maxq,
                          Sq=int(rng.integers(1, maxq + 1)), L=[int(x) for x in rng.integers(0, 4000, B)],
                          page=int(rng.choice([0, 0, 16, 64, 256])), s_new=int(rng.choice([0, 0, 1])),
                          causal=causal, window=window, softcap=float(rng.choice([0.0, 0.0, 10.0])),
                          num_splits=int(rng.choice([0, 0, 1, 3])), pack_gqa=[None, False][int(rng.random() < 0.3)],
                          dtype=str(rng.choice(["bf16", "fp16"])), seed=7000 + i))
    return cases


MD_CASES = _md_cases(60, 20251208)


@pytest.mark.parametrize("i", range(len(MD_CASES)))
def test_random_scheduler_metadata(i):
    import torch
    from flash_attn_npu_v3 import flash_attn_with_kvcache, get_scheduler_metadata
    from tests._util import bits, randn
    c = MD_CASES[i]
    print(f"case random scheduler metadata {i}: {c}", flush=True)
    dt = _dt(c["dtype"])
    B, H, Hk, D, Sq, page, s_new = c["B"], c["H"], c["Hk"], c["D"], c["Sq"], c["page"], c["s_new"]
    g = torch.Generator().manual_seed(c["seed"])
    L = np.asarray(c["L"], np.int32)
    if page:
        need = [(int(x) + s_new + page - 1) // page for x in L]
        nb = sum(need) + 3
        perm = torch.randperm(nb, generator=g).to(torch.int32)
        bt = torch.zeros((B, max(max(need), 1)), dtype=torch.int32)
        o = 0
        for b in range(B):
            bt[b, :need[b]] = perm[o:o + need[b]]
            o += need[b]
        kc, vc = randn((nb, page, Hk, D), dt, g, "cpu"), randn((nb, page, Hk, D), dt, g, "cpu")
        max_k = bt.shape[1] * page
    else:
        bt = None
        max_k = int(L.max()) + s_new + 8
        kc, vc = randn((B, max_k, Hk, D), dt, g, "cpu"), randn((B, max_k, Hk, D), dt, g, "cpu")
    q = randn((B, Sq, H, D), dt, g, "cpu")
    kn = vn = None
    if s_new:
        kn, vn = randn((B, s_new, Hk, D), dt, g, "cpu"), randn((B, s_new, Hk, D), dt, g, "cpu")
    sl = torch.from_numpy(L).to("cuda")
    md = get_scheduler_metadata(B, c["maxq"], max_k, H, Hk, D, sl, qkv_dtype=dt, page_size=page or None,
                                max_seqlen_k_new=s_new, causal=c["causal"], window_size=c["window"],
                                has_softcap=c["softcap"] > 0, num_splits=c["num_splits"], pack_gqa=c["pack_gqa"])
    res = []
    for use in (True, False):
        kcd, vcd = kc.to("cuda"), vc.to("cuda")
        d = lambda x: None if x is None else x.to("cuda")
        o, lse, *_ = flash_attn_with_kvcache(d(q), kcd, vcd, k=d(kn), v=d(vn), cache_seqlens=sl, page_table=d(bt),
                                             causal=c["causal"], window_size=c["window"], softcap=c["softcap"],
                                             num_splits=c["num_splits"], pack_gqa=c["pack_gqa"],
                                             return_softmax_lse=True, scheduler_metadata=md if use else None)
        torch.cuda.synchronize()
        res.append((bits(o), lse.cpu().numpy().view(np.uint32), bits(kcd), bits(vcd)))
    for a, b in zip(*res):
        assert np.array_equal(a, b), "the call with scheduler_metadata differs from the call without it"
