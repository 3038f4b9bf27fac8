#!/usr/bin/env python3
"""Benchmark of the MI355X FlashAttention forward path on the BASELINE configs.

One JSON line on stdout. The headline (`value`) is BASELINE config 2 -- the
contiguous-KV GQA decode with a 1-token in-place append (B=32, H=32/8, D=128,
bf16, caches (32, 8192, 8, 128), cache_seqlens ~ U[1024, 8191]) -- as
algorithmic HBM TB/s of the whole call (append + attention + combine), inputs
resident in HBM. Configs 3-5 are reported in `configs` beside it; config 1 is
the CPU-runnable parity anchor and is not a bench line.

Every call goes through the C ABI (libfa_mi355x.so via ctypes); PyTorch only
allocates device memory and supplies the stream. Kernel durations come from
HIP events recorded by the library at stage boundaries (fa_fwd_params.
stage_events) on the stream the kernels run on. Each stage also carries the
cost of its event packets (a few us; `event_pair_us` where a config has no
append kernel and the append stage is empty), so stage times are upper bounds
of the kernel durations that a rocprofv3 kernel trace gives. Caches are rotated between
copies so reads are not served by the 256 MB Infinity Cache. Each config
gets W untimed warmup calls, then untimed calls for about 150 ms more (the
shader clock ramps up after the idle gap spent building the config's inputs),
then exactly K timed calls.

Each of configs 2-5 also carries a `parity` block: one more call on the
benchmarked inputs, compared with the oracle's result on the cpu_baseline
sample (out max-abs, LSE relative error, the cache after the append bit for
bit); the headline's is repeated at the top level.

`configs` also carries "bwd", the backward of a dense causal training shape,
and "c2f8" / "c3f8", configs 2 and 3 with q, the caches and the new k/v in
float8_e4m3fn (bf16 out); none of these is a BASELINE config.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c2,c3,c4,c5,bwd,c2f8,c3f8] [--no-cpu]
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "flash-attention-npu_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
METRIC = "decode attn µs/call + achieved HBM TB/s; prefill TFLOP/s (% bf16 MFMA peak)"


# ---- HIP events through the runtime's C API --------------------------------------------------
class Hip:
    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]

    def event(self):
        e = ctypes.c_void_p()
        assert self.lib.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def record(self, e, stream):
        assert self.lib.hipEventRecord(e, stream) == 0

    def ms(self, a, b):
        assert self.lib.hipEventSynchronize(b) == 0
        out = ctypes.c_float()
        assert self.lib.hipEventElapsedTime(ctypes.byref(out), a, b) == 0
        return out.value


# ---- config builders --------------------------------------------------------------------------
def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def build_case(name, torch, dev, ncopy):
    """Returns dict with per-copy C-ABI params, algorithmic work, host slices for the CPU baseline."""
    from fa_mi355x import capi
    g = torch.Generator(device=dev)
    gc = torch.Generator()
    bf = torch.bfloat16
    D = 128
    keep = []

    # "c2f8" / "c3f8": the same workloads with q, the caches and k/v in
    # float8_e4m3fn (N(0,1) values rounded to e4m3, unit descales), out bf16
    f8 = name.endswith("f8")
    base = name[:-2] if f8 else name

    def rn(*shape):
        t = torch.randn(shape, generator=g, device=dev, dtype=torch.float32)
        return t.to(torch.float8_e4m3fn) if f8 else t.to(bf)

    c = {"name": name}
    if base == "c2":
        g.manual_seed(2); gc.manual_seed(2)
        B, Sq, H, Hk, cap = 32, 1, 32, 8, 8192
        L = torch.randint(1024, 8192, (B,), generator=gc, dtype=torch.int32)
        q, kn, vn = rn(B, Sq, H, D), rn(B, 1, Hk, D), rn(B, 1, Hk, D)
        caches = [(rn(B, cap, Hk, D), rn(B, cap, Hk, D)) for _ in range(ncopy)]
        bt = None
        bidx = None
        window, alibi, cos, sin = (-1, -1), None, None, None
        s_new = 1
        kv_tokens = int((L + 1).sum())
        c["work_desc"] = "B32 Sq1 H32/8 D128 bf16 contiguous cache 32x8192, L~U[1024,8191], 1-token append"
    elif base == "c3":
        g.manual_seed(3); gc.manual_seed(3)
        B, Sq, H, Hk, page = 64, 1, 64, 8, 256
        L = torch.round(torch.exp(torch.empty(B).uniform_(math.log(512), math.log(32768), generator=gc))).to(torch.int32)
        need = ((L + 1 + page - 1) // page).tolist()
        nblocks = int(sum(int(math.ceil(int(x) / page)) for x in L) * 1.1) + 1
        nblocks = max(nblocks, sum(need))
        perm = torch.randperm(nblocks, generator=gc).to(torch.int32)
        maxb = max(need)
        bt_h = torch.zeros((B, maxb), dtype=torch.int32)
        o = 0
        for b in range(B):
            bt_h[b, :need[b]] = perm[o:o + need[b]]
            o += need[b]
        bt = bt_h.to(dev)
        q, kn, vn = rn(B, Sq, H, D), rn(B, 1, Hk, D), rn(B, 1, Hk, D)
        caches = [(rn(nblocks, page, Hk, D), rn(nblocks, page, Hk, D)) for _ in range(ncopy)]
        bidx = None
        window, alibi, cos, sin = (-1, -1), None, None, None
        s_new = 1
        kv_tokens = int((L + 1).sum())
        cap = maxb * page
        c["work_desc"] = "B64 Sq1 H64/8 D128 bf16 paged(256) permuted block_table, L log-uniform [512,32768], 1-token append"
    elif base == "c4":
        g.manual_seed(4); gc.manual_seed(4)
        B, Sq, H, Hk, cap = 4, 2048, 32, 8, 8192
        L = torch.full((B,), 6144, dtype=torch.int32)
        q, kn, vn = rn(B, Sq, H, D), rn(B, Sq, Hk, D), rn(B, Sq, Hk, D)
        caches = [(rn(B, cap, Hk, D), rn(B, cap, Hk, D)) for _ in range(ncopy)]
        inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
        ang = torch.arange(cap, dtype=torch.float32)[:, None] * inv[None, :]
        cos, sin = torch.cos(ang).to(bf).to(dev), torch.sin(ang).to(bf).to(dev)
        bt = None
        bidx = None
        window, alibi = (-1, -1), None
        s_new = Sq
        kv_tokens = None
        c["work_desc"] = "B4 2048 new tokens onto 6144 cached (cache 8192), H32/8 D128 bf16, NeoX rotary, causal"
    elif name == "c5":
        g.manual_seed(5); gc.manual_seed(5)
        B, Sq, H, Hk, page = 8, 4, 32, 8, 256
        L = torch.randint(16384, 65537, (B,), generator=gc, dtype=torch.int32)
        bidx_h = torch.randperm(B, generator=gc).to(torch.int32)
        need_rows = [0] * B
        for b in range(B):
            need_rows[int(bidx_h[b])] = (int(L[b]) + page - 1) // page
        nblocks = int(sum(need_rows) * 1.1) + 1
        perm = torch.randperm(nblocks, generator=gc).to(torch.int32)
        maxb = max(need_rows)
        bt_h = torch.zeros((B, maxb), dtype=torch.int32)
        o = 0
        for r in range(B):
            bt_h[r, :need_rows[r]] = perm[o:o + need_rows[r]]
            o += need_rows[r]
        bt = bt_h.to(dev)
        bidx = bidx_h.to(dev)
        q = rn(B, Sq, H, D)
        kn = vn = None
        caches = [(rn(nblocks, page, Hk, D), rn(nblocks, page, Hk, D)) for _ in range(ncopy)]
        window = (4096, 0)
        alibi = torch.tensor([2.0 ** (-8.0 * (h + 1) / H) for h in range(H)], dtype=torch.float32, device=dev)
        cos = sin = None
        s_new = 0
        kv_tokens = None
        cap = maxb * page
        c["work_desc"] = "B8 Sq4 H32/8 D128 bf16 paged(256), L~U[16384,65536], cache_batch_idx perm, window (4096,0), ALiBi"
    else:
        raise ValueError(name)

    sl = L.to(dev)
    out = torch.empty((B, Sq, H, D), dtype=bf, device=dev)
    lse = torch.empty((B, H, Sq), dtype=torch.float32, device=dev)
    params = []
    for (kc, vc) in caches:
        p = capi.new_params(
            dtype=capi.FA_DTYPE_FP8_E4M3 if f8 else capi.FA_DTYPE_BF16, batch=B, seqlen_q=Sq, nheads=H,
            nheads_k=Hk, headdim=D, headdim_v=D,
            seqlen_k=kc.shape[1] if bt is None else 0, batch_cache=kc.shape[0],
            q=_ptr(q), q_batch_stride=q.stride(0), q_row_stride=q.stride(1), q_head_stride=q.stride(2),
            k=_ptr(kc), k_batch_stride=kc.stride(0), k_row_stride=kc.stride(1), k_head_stride=kc.stride(2),
            v=_ptr(vc), v_batch_stride=vc.stride(0), v_row_stride=vc.stride(1), v_head_stride=vc.stride(2),
            out=_ptr(out), out_batch_stride=out.stride(0), out_row_stride=out.stride(1),
            out_head_stride=out.stride(2), softmax_lse=_ptr(lse), cache_seqlens=_ptr(sl),
            softmax_scale=D ** -0.5, is_causal=1, window_size_left=window[0], window_size_right=window[1])
        if kn is not None:
            p.k_new, p.v_new = _ptr(kn), _ptr(vn)
            p.knew_batch_stride, p.knew_row_stride, p.knew_head_stride = kn.stride(0), kn.stride(1), kn.stride(2)
            p.vnew_batch_stride, p.vnew_row_stride, p.vnew_head_stride = vn.stride(0), vn.stride(1), vn.stride(2)
            p.seqlen_new = s_new
        if bt is not None:
            p.block_table = _ptr(bt)
            p.block_table_batch_stride = bt.stride(0)
            p.max_blocks_per_seq = bt.shape[1]
            p.block_table_rows = bt.shape[0]
            p.page_block_size = kc.shape[1]
        if bidx is not None:
            p.cache_batch_idx = _ptr(bidx)
        if cos is not None:
            p.rotary_cos, p.rotary_sin = _ptr(cos), _ptr(sin)
            p.rotary_dim, p.seqlen_ro, p.rotary_interleaved = 2 * cos.shape[1], cos.shape[0], 0
        if alibi is not None:
            p.alibi_slopes = _ptr(alibi)
        st, nbytes = capi.workspace_size(p, capi.FA_KIND_KVCACHE)
        assert st == 0, capi.last_error()
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
        keep.append(ws)
        p.workspace, p.workspace_bytes = _ptr(ws), ws.numel()
        params.append(p)

    if f8:
        c["work_desc"] = c["work_desc"].replace("bf16", "fp8 e4m3 (q, cache, k/v; bf16 out)")
    # algorithmic work (per call)
    e = 1 if f8 else 2
    if base in ("c2", "c3"):
        kv = 2 * kv_tokens * Hk * D * e                      # K and V of L+1 tokens
        qo = B * Sq * H * D * (e + 2) + 4 * B * H * Sq        # q read, bf16 out write, lse write
        app = 2 * 2 * B * Hk * D * e                          # new k/v read + cache write
        c["attn_bytes"] = kv + qo
        c["bytes"] = kv + qo + app
        c["bound"] = "hbm"
    elif name == "c5":
        keys = 0
        for b in range(B):
            Lb = int(L[b])
            lo = max(0, Lb - Sq - 4096)     # union of the 4 rows' windows
            keys += Lb - lo
        c["attn_bytes"] = 2 * keys * Hk * D * e + 2 * B * Sq * H * D * e + 4 * B * H * Sq
        c["bytes"] = c["attn_bytes"]
        c["bound"] = "hbm"
    else:  # c4
        P = sum(6145 + i for i in range(2048))
        c["flops"] = 4 * D * P * B * H
        c["bound"] = "mfma"
    c.update(params=params, keep=[q, kn, vn, caches, bt, bidx, cos, sin, alibi, out, lse, sl],
             B=B, Sq=Sq, H=H, Hk=Hk, L=L)
    return c


WARM_MS = 150.0


def time_case(c, hip, torch, steps, warmup):
    from fa_mi355x import capi
    L = capi.lib()
    stream = torch.cuda.current_stream().cuda_stream
    ps = c["params"]
    n = len(ps)

    def call(i, ev=None):
        p = ps[i % n]
        p.stage_events = ev
        st = L.fa_mha_fwd_kvcache(ctypes.byref(p), stream)
        if st != 0:
            raise RuntimeError(capi.last_error())

    for i in range(warmup):
        call(i)
    torch.cuda.synchronize()
    # After an idle gap (building the next config's inputs) the shader clock
    # ramps back up over tens of milliseconds, which shows in the compute-bound
    # prefill (c4). The W warmup calls are therefore followed by more untimed
    # calls until about WARM_MS of GPU time has passed.
    t0 = time.perf_counter()
    call(warmup)
    torch.cuda.synchronize()
    one_ms = (time.perf_counter() - t0) * 1e3
    extra = min(int(WARM_MS / max(one_ms, 1e-3)), 2000)
    for i in range(extra):
        call(warmup + 1 + i)
    torch.cuda.synchronize()
    # pass 1: whole calls, back to back
    a, b = hip.event(), hip.event()
    hip.record(a, stream)
    for i in range(steps):
        call(i)
    hip.record(b, stream)
    whole_ms = hip.ms(a, b) / steps
    torch.cuda.synchronize()
    # pass 2: per-stage events (append | attention | combine)
    evs = [[hip.event() for _ in range(4)] for _ in range(steps)]
    arrs = [(ctypes.c_void_p * 4)(*[e.value for e in ev]) for ev in evs]
    for i in range(steps):
        call(i, ctypes.cast(arrs[i], ctypes.c_void_p))
    torch.cuda.synchronize()
    st = [[hip.ms(ev[k], ev[k + 1]) for k in range(3)] for ev in evs]
    mean = lambda xs: sum(xs) / len(xs)
    return {"us_per_call": whole_ms * 1e3,
            "append_us": mean([s[0] for s in st]) * 1e3,
            "attn_us": mean([s[1] for s in st]) * 1e3,
            "combine_us": mean([s[2] for s in st]) * 1e3}


CPU_BUDGET_S = 10.0   # wall time per config for the CPU golden


def _cpu_threads():
    return min(16, os.cpu_count() or 1)


def _timed(fn):
    """Runs fn until CPU_BUDGET_S has passed (at least once);
    returns (seconds per run, runs)."""
    t0 = time.perf_counter()
    reps = 0
    while True:
        fn()
        reps += 1
        if time.perf_counter() - t0 > CPU_BUDGET_S or reps >= 1000:
            break
    return (time.perf_counter() - t0) / reps, reps


def cpu_baseline(c, torch):
    """The oracle (the C restatement of the reference golden,
    tests/test_flash_attn_npu_v3.py:87-146 of the reference) on the host cores,
    on a bounded sample of the config's own inputs, in the config's unit:
      c2 / c3: the first sequences (all heads), TB/s of the same algorithmic bytes;
      c4: one (batch, kv head) slice (its 4 query heads, rotary and append), TFLOP/s;
      c5: the whole config, TB/s.
    Returns (baseline, ref): ref holds the oracle's out / LSE / caches after the
    append for that sample, which parity() compares with the GPU's."""
    import numpy as np
    from oracle import fa_oracle as orc
    nt = _cpu_threads()
    name = c["name"]
    q, kn, vn, caches, bt, bidx, cos, sin, alibi = c["keep"][:9]
    kc, vc = caches[0]
    L = c["L"]
    H, Hk, D = c["H"], c["Hk"], 128
    bits = lambda t: t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
    if name in ("c2", "c3"):
        nb = 8 if name == "c2" else 4
        qh, knh, vnh = bits(q[:nb]), bits(kn[:nb]), bits(vn[:nb])
        if bt is None:
            kh, vh, bth = bits(kc[:nb]), bits(vc[:nb]), None
        else:  # the pages the sample's sequences use, renumbered
            rows = bt[:nb].cpu()
            used = torch.unique(rows)
            remap = torch.zeros(int(used.max()) + 1, dtype=torch.int32)
            remap[used.long()] = torch.arange(used.numel(), dtype=torch.int32)
            kh, vh = bits(kc[used.to(kc.device).long()]), bits(vc[used.to(vc.device).long()])
            bth = remap[rows.long()].numpy()
        Ls = L[:nb]
        res = {}

        def run():
            res["r"] = orc.kvcache_forward(qh, kh, vh, dtype=orc.BF16, cache_seqlens=Ls.numpy(), k=knh, v=vnh,
                                           block_table=bth, causal=True, nthreads=nt)
        dt, reps = _timed(run)
        nbytes = 2 * int((Ls + 1).sum()) * Hk * D * 2 + 2 * nb * H * D * 2 + 4 * nb * H + 2 * 2 * nb * Hk * D * 2
        sample = f"config {name[1]}, sequences 0..{nb - 1} of {c['B']} (all {H} q heads)"
        ro, rl, rk, rv = res["r"]
        sel_kv = (lambda t: t[:nb]) if bt is None else (lambda t: t[used.to(t.device).long()])
        ref = {"out": ro, "lse": rl, "k": rk, "v": rv, "sel_q": lambda t: t[:nb], "sel_kv": sel_kv,
               "sample": sample + ("" if bt is None else ", the cache pages they use")}
        return ({"value": round(nbytes / dt / 1e12, 6), "unit": "TB/s", "cores": nt, "host_cores": os.cpu_count(),
                 "kind": "port", "sample": f"{sample}, oracle/fa_oracle.c on {nt} OpenMP threads, {reps} reps, "
                 f"{dt * 1e3:.1f} ms/rep"}, ref)
    if name == "c4":
        g = H // Hk
        qh = bits(q[0:1, :, 0:g])
        kh, vh = bits(kc[0:1, :, 0:1]), bits(vc[0:1, :, 0:1])
        knh, vnh = bits(kn[0:1, :, 0:1]), bits(vn[0:1, :, 0:1])
        ch, sh = bits(cos), bits(sin)
        res = {}

        def run():
            res["r"] = orc.kvcache_forward(qh, kh, vh, dtype=orc.BF16, cache_seqlens=L[0:1].numpy(), k=knh, v=vnh,
                                           rotary_cos=ch, rotary_sin=sh, rotary_interleaved=False, causal=True,
                                           nthreads=nt)
        dt, reps = _timed(run)
        flops = c["flops"] / (c["B"] * H) * g
        sample = f"config 4, batch 0 x kv head 0 (q heads 0..{g - 1}): 1/{c['B'] * Hk} of the work"
        ro, rl, rk, rv = res["r"]
        ref = {"out": ro, "lse": rl, "k": rk, "v": rv, "sel_q": lambda t: t[0:1, :, 0:g] if t.dim() == 4 else t[0:1, 0:g],
               "sel_kv": lambda t: t[0:1, :, 0:1], "sample": sample + ", its whole cache after the append"}
        return ({"value": round(flops / dt / 1e12, 6), "unit": "TFLOP/s", "cores": nt, "host_cores": os.cpu_count(),
                 "kind": "port", "sample": f"{sample}, oracle/fa_oracle.c on {nt} OpenMP threads, {reps} reps, "
                 f"{dt * 1e3:.0f} ms/rep"}, ref)
    # c5: the whole config
    qh, kh, vh = bits(q), bits(kc), bits(vc)
    res = {}

    def run():
        res["r"] = orc.kvcache_forward(qh, kh, vh, dtype=orc.BF16, cache_seqlens=L.numpy(),
                                       cache_batch_idx=bidx.cpu().numpy(), block_table=bt.cpu().numpy(), causal=True,
                                       window=(4096, 0), alibi=alibi.cpu().numpy(), nthreads=nt)
    dt, reps = _timed(run)
    ro, rl, _, _ = res["r"]
    ref = {"out": ro, "lse": rl, "k": None, "v": None, "sel_q": lambda t: t, "sel_kv": None,
           "sample": f"config 5, all {c['B']} sequences (no append)"}
    return ({"value": round(c["attn_bytes"] / dt / 1e12, 6), "unit": "TB/s", "cores": nt,
             "host_cores": os.cpu_count(), "kind": "port",
             "sample": f"config 5, all {c['B']} sequences, oracle/fa_oracle.c on {nt} OpenMP threads, {reps} reps, "
                       f"{dt * 1e3:.1f} ms/rep"}, ref)


def parity(c, ref, torch):
    """The GPU's result on the benchmarked inputs against the oracle's on the
    cpu_baseline sample: one more call on the first cache copy (the one the
    oracle ran on), then out max-abs against the bf16 bar of 1e-2 (plus one
    ulp of the reference value: both outputs are rounded to bf16 from their
    fp32 values), LSE relative error against 1e-4 (with a 1e-5 absolute floor for
    |LSE| < 0.1), and the cache after the append bit for bit."""
    import numpy as np
    from fa_mi355x import capi
    from oracle import fa_oracle as orc
    q, kn, vn, caches, bt, bidx, cos, sin, alibi, out, lse = c["keep"][:11]
    p = c["params"][0]
    p.stage_events = None
    st = capi.lib().fa_mha_fwd_kvcache(ctypes.byref(p), torch.cuda.current_stream().cuda_stream)
    if st != 0:
        raise RuntimeError(capi.last_error())
    torch.cuda.synchronize()
    bits = lambda t: t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
    got = ref["sel_q"](out).float().cpu().numpy()
    want = orc.from_bits(ref["out"], orc.BF16).reshape(got.shape)
    err = np.abs(got - want)
    out_ok = bool((err <= 1e-2 + np.abs(want) * 2.0 ** -7).all()) and not np.isnan(got).any()
    gl = ref["sel_q"](lse).cpu().numpy().astype(np.float64)
    rl = np.asarray(ref["lse"], dtype=np.float64).reshape(gl.shape)
    fin = np.isfinite(rl)
    dl = np.abs(gl[fin] - rl[fin])
    lse_ok = bool(np.array_equal(np.isinf(gl), np.isinf(rl)) and (dl <= 1e-4 * np.abs(rl[fin]) + 1e-5).all())
    r = {"out_max_abs": float(err.max()), "out_tol": 1e-2, "lse_max_rel": float((dl / np.abs(rl[fin])).max()),
         "lse_tol_rel": 1e-4, "sample": ref["sample"]}
    if ref["k"] is not None:
        kc, vc = caches[0]
        r["cache_bit_exact"] = bool(np.array_equal(bits(ref["sel_kv"](kc)), ref["k"]) and
                                    np.array_equal(bits(ref["sel_kv"](vc)), ref["v"]))
    else:
        r["cache_bit_exact"] = None
    r["ok"] = out_ok and lse_ok and r["cache_bit_exact"] is not False
    return r


# The matrix-core issue rate without memory: every wave runs chains of
# independent bf16 MFMAs on register operands (8 accumulators of 16x16x32, or
# 4 of 32x32x16), two waves per SIMD, one workgroup per CU.
_MFMA_PROBE_SRC = r"""
#include <hip/hip_runtime.h>
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
template <int KIND>
__global__ void __launch_bounds__(512) mfma_probe(float* out, int iters, float seed) {
    bf16x8 a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = (__bf16)(seed * (float)(threadIdx.x + i));
        b[i] = (__bf16)(seed * (float)(i + 1));
    }
    float s = 0.f;
    if constexpr (KIND == 0) {
        f32x4 acc[8];
        for (int j = 0; j < 8; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[j], 0, 0, 0);
        }
        for (int j = 0; j < 8; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
    } else {
        f32x16 acc[4];
        for (int j = 0; j < 4; ++j) acc[j] = f32x16{};
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
        }
        for (int j = 0; j < 4; ++j)
            for (int e = 0; e < 16; ++e) s += acc[j][e];
    }
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}
extern "C" int fa_mfma_probe(int kind, int blocks, int iters, float* out, void* stream) {
    if (kind == 0) hipLaunchKernelGGL(mfma_probe<0>, dim3(blocks), dim3(512), 0, (hipStream_t)stream, out, iters, 1e-3f);
    else hipLaunchKernelGGL(mfma_probe<1>, dim3(blocks), dim3(512), 0, (hipStream_t)stream, out, iters, 1e-3f);
    return (int)hipGetLastError();
}
"""


def mfma_rate(torch, hip, timed):
    """bf16 TFLOP/s of the MFMA probe above (built here with hipcc, in a
    temporary directory), 16x16x32 and 32x32x16."""
    import subprocess
    import tempfile
    res = {}
    with tempfile.TemporaryDirectory() as d:
        src, lib = os.path.join(d, "mfma_probe.hip"), os.path.join(d, "mfma_probe.so")
        with open(src, "w") as f:
            f.write(_MFMA_PROBE_SRC)
        subprocess.run(["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O3", "-shared", "-fPIC", "-Xclang",
                        "-target-feature", "-Xclang", "-packed-fp32-ops", src, "-o", lib], check=True,
                       capture_output=True)
        probe = ctypes.CDLL(lib)
        probe.fa_mfma_probe.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        cus = torch.cuda.get_device_properties(0).multi_processor_count
        out = torch.empty(cus * 512, dtype=torch.float32, device="cuda")
        stream = torch.cuda.current_stream().cuda_stream
        iters = 4000
        for kind, name, flop in ((0, "mfma_16x16x32_bf16_tflops", 8 * 16384), (1, "mfma_32x32x16_bf16_tflops", 4 * 32768)):
            def run():
                if probe.fa_mfma_probe(kind, cus, iters, out.data_ptr(), stream) != 0:
                    raise RuntimeError("MFMA probe launch failed")
            t = timed(run, 5)
            res[name] = round(cus * 8 * iters * flop / t / 1e12, 1)
    return res


# A read-only copy of the decode kernel's loads: the same tile list (32-key
# tiles of every (sequence, kv head) segment, visible keys only), the same
# per-lane 16-byte chunks (16 key rows x 64 contiguous bytes per load
# instruction), 4 waves per CU with an equal split of the tiles, the waves of
# a CU streaming adjacent kv heads of one range (4 heads when the kv head count
# is a multiple of 4, else 2 when it is even), 3 tiles in flight, no compute (an xor of every load). Its time is the rate HBM gives
# that access pattern, the decode kernel's own ceiling.
_DECODE_READ_SRC = r"""
#include <hip/hip_runtime.h>
#include <stdint.h>
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int MAXB = 64, HKM = 8;
struct RdArgs {
    const uint16_t* k; const uint16_t* v; const int* bt; long long bt_stride; int nblocks, page;
    const int* pref; const int* lot; const int* sk; const int* crow; int B, Hk;
    long long sb, si, sh; u32x4* sink;
};
__global__ void __launch_bounds__(256, 1) decode_read(RdArgs a) {
    __shared__ int s_pref[MAXB + 1], s_lot[MAXB], s_sk[MAXB], s_crow[MAXB];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, G = lane >> 4;
    if (tid <= a.B) s_pref[tid] = a.pref[tid];
    if (tid < a.B) { s_lot[tid] = a.lot[tid]; s_sk[tid] = a.sk[tid]; s_crow[tid] = a.crow[tid]; }
    __syncthreads();
    const int T = s_pref[a.B];
    // the decode kernel's worker groups: the 4 (or 2) waves of a group take one
    // tile range of kv head groups, each wave one head of the group
    const int hs = (a.Hk % 4) == 0 ? 4 : ((a.Hk % 2) == 0 ? 2 : 1), hsel = wave % hs;
    const long long W = (long long)gridDim.x * (4 / hs), gw = (long long)(wave / hs) * gridDim.x + blockIdx.x;
    const long long wid = gw * hs + hsel;
    const int t0 = (int)(gw * T / W), t1 = (int)((gw + 1) * T / W);
    u32x4 kr[3][2][4], vr[3][2][4];
    u32x4 acc = {0u, 0u, 0u, 0u};
    auto issue = [&](int t, u32x4 (&kk)[2][4], u32x4 (&vv)[2][4]) {
        if (t >= t1) return;
        int bl = 0, bh = a.B;
        while (bh - bl > 1) { const int m = (bl + bh) >> 1; if (s_pref[m] <= t) bl = m; else bh = m; }
        const int per = (s_pref[bl + 1] - s_pref[bl]) / (a.Hk / hs), o = t - s_pref[bl];
        const int hk = (o / per) * hs + hsel, j = o % per, sk = s_sk[bl];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            int key = (s_lot[bl] + j) * 32 + h * 16 + li;
            key = key < sk ? key : sk - 1;
            long long off;
            if (a.bt) {
                int blk = a.bt[(long long)s_crow[bl] * a.bt_stride + key / a.page];
                blk = blk < 0 ? 0 : (blk >= a.nblocks ? a.nblocks - 1 : blk);
                off = (long long)blk * a.sb + (long long)(key % a.page) * a.si + (long long)hk * a.sh;
            } else {
                off = (long long)s_crow[bl] * a.sb + (long long)key * a.si + (long long)hk * a.sh;
            }
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                kk[h][s] = *reinterpret_cast<const u32x4*>(a.k + off + 8 * (4 * s + G));
                vv[h][s] = *reinterpret_cast<const u32x4*>(a.v + off + 8 * (4 * s + G));
            }
        }
    };
    issue(t0, kr[0], vr[0]);
    issue(t0 + 1, kr[1], vr[1]);
    for (int tb = t0; tb < t1; tb += 3) {
#pragma unroll
        for (int st = 0; st < 3; ++st) {
            const int t = tb + st;
            if (t < t1) {
                issue(t + 2, kr[(st + 2) % 3], vr[(st + 2) % 3]);
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int s = 0; s < 4; ++s) acc ^= kr[st][h][s] ^ vr[st][h][s];
            }
        }
    }
    a.sink[wid * 64 + lane] = acc;
}
extern "C" int fa_decode_read(const RdArgs* a, int grid, void* stream) {
    if (a->B > MAXB) return 1;
    hipLaunchKernelGGL(decode_read, dim3(grid), dim3(256), 0, (hipStream_t)stream, *a);
    return (int)hipGetLastError();
}
"""


class _RdArgs(ctypes.Structure):
    _fields_ = [("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("bt", ctypes.c_void_p),
                ("bt_stride", ctypes.c_longlong), ("nblocks", ctypes.c_int), ("page", ctypes.c_int),
                ("pref", ctypes.c_void_p), ("lot", ctypes.c_void_p), ("sk", ctypes.c_void_p),
                ("crow", ctypes.c_void_p), ("B", ctypes.c_int), ("Hk", ctypes.c_int),
                ("sb", ctypes.c_longlong), ("si", ctypes.c_longlong), ("sh", ctypes.c_longlong),
                ("sink", ctypes.c_void_p)]


def decode_read_ceiling(torch, hip, timed):
    """Microseconds per call of the read-only copy of the decode kernel's loads
    above on the inputs of configs c2 and c5 (the same caches, rotated the same
    way), against the decode kernel's own attention time on them."""
    import subprocess
    import tempfile
    res = {}
    with tempfile.TemporaryDirectory() as d:
        src, lib = os.path.join(d, "decode_read.hip"), os.path.join(d, "decode_read.so")
        with open(src, "w") as f:
            f.write(_DECODE_READ_SRC)
        subprocess.run(["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O3", "-shared", "-fPIC", "-Xclang",
                        "-target-feature", "-Xclang", "-packed-fp32-ops", src, "-o", lib], check=True,
                       capture_output=True)
        probe = ctypes.CDLL(lib)
        probe.fa_decode_read.argtypes = [ctypes.POINTER(_RdArgs), ctypes.c_int, ctypes.c_void_p]
        cus = torch.cuda.get_device_properties(0).multi_processor_count
        stream = torch.cuda.current_stream().cuda_stream
        sink = torch.empty(cus * 4 * 64 * 4, dtype=torch.int32, device="cuda")
        for name, ncopy in (("c2", 2), ("c5", 4)):
            c = build_case(name, torch, "cuda", ncopy)
            q, kn, vn, caches, bt, bidx = c["keep"][:6]
            B, Hk, Sq = c["B"], c["Hk"], c["Sq"]
            L = [int(x) for x in c["L"]]
            if name == "c2":
                sk, lo = [x + 1 for x in L], [0] * B          # the cached keys and the appended one
                crow = list(range(B))
            else:
                sk, lo = L, [max(0, x - Sq - 4096) for x in L]  # the union of the 4 rows' windows
                crow = [int(x) for x in bidx.cpu()]
            lot = [x // 32 for x in lo]
            pref = [0]  # tile prefix over (sequence, kv head group)
            groups = Hk // 4 if Hk % 4 == 0 else (Hk // 2 if Hk % 2 == 0 else Hk)
            for b in range(B):
                pref.append(pref[-1] + groups * ((sk[b] + 31) // 32 - lot[b]))
            ints = {n_: torch.tensor(v_, dtype=torch.int32, device="cuda")
                    for n_, v_ in (("pref", pref), ("lot", lot), ("sk", sk), ("crow", crow))}
            args = []
            for kc, vc in caches:
                assert kc.stride() == vc.stride() and kc.shape[-1] == 128
                a = _RdArgs(k=kc.data_ptr(), v=vc.data_ptr(), bt=0 if bt is None else bt.data_ptr(),
                            bt_stride=0 if bt is None else bt.stride(0), nblocks=kc.shape[0],
                            page=kc.shape[1] if bt is not None else 1, pref=ints["pref"].data_ptr(),
                            lot=ints["lot"].data_ptr(), sk=ints["sk"].data_ptr(), crow=ints["crow"].data_ptr(),
                            B=B, Hk=Hk, sb=kc.stride(0), si=kc.stride(1), sh=kc.stride(2), sink=sink.data_ptr())
                args.append(a)
            state = {"i": 0}

            def run():
                a = args[state["i"] % len(args)]
                state["i"] += 1
                if probe.fa_decode_read(ctypes.byref(a), cus, stream) != 0:
                    raise RuntimeError("decode read probe launch failed")
            t = timed(run, 40)
            res[f"decode_read_only_{name}_us"] = round(t * 1e6, 1)
            res[f"decode_read_only_{name}_tbps"] = round(c["attn_bytes"] / t / 1e12, 3)
            del c, args, ints
            torch.cuda.empty_cache()
    return res


def ceilings(torch, hip):
    """Practical ceilings of this part: HBM bandwidth of a 4 GiB device copy
    (read + write) and of a 4 GiB reduction (read), bf16 TFLOP/s of a large
    GEMM (torch.matmul, hipBLASLt) and of the MFMA issue rate alone."""
    stream = torch.cuda.current_stream().cuda_stream
    res = {}

    def timed(fn, n):
        fn()
        torch.cuda.synchronize()
        a, b = hip.event(), hip.event()
        hip.record(a, stream)
        for _ in range(n):
            fn()
        hip.record(b, stream)
        return hip.ms(a, b) / n * 1e-3

    x = torch.empty(1 << 31, dtype=torch.bfloat16, device="cuda").normal_()
    y = torch.empty_like(x)
    t = timed(lambda: y.copy_(x), 10)
    res["hbm_copy_tbps"] = round(2 * x.numel() * 2 / t / 1e12, 3)
    acc = torch.empty((), dtype=torch.float32, device="cuda")
    t = timed(lambda: torch.sum(x, dim=0, dtype=torch.float32, out=acc), 10)
    res["hbm_read_tbps"] = round(x.numel() * 2 / t / 1e12, 3)
    del x, y
    n = 8192
    a = torch.randn((n, n), device="cuda").to(torch.bfloat16)
    b = torch.randn((n, n), device="cuda").to(torch.bfloat16)
    c = torch.empty((n, n), device="cuda", dtype=torch.bfloat16)
    for _ in range(20):
        torch.matmul(a, b, out=c)  # clock warm-up
    t = timed(lambda: torch.matmul(a, b, out=c), 50)
    res["gemm_bf16_tflops"] = round(2 * n ** 3 / t / 1e12, 1)
    del a, b, c
    res.update(mfma_rate(torch, hip, timed))
    res.update(decode_read_ceiling(torch, hip, timed))
    res["note"] = ("4 GiB bf16 copy (2 x 4 GiB moved), torch.sum of 4 GiB bf16, 8192^3 bf16 torch.matmul, "
                   "register-only bf16 MFMA chains (2 waves per SIMD, 8 x 16x16x32 or 4 x 32x32x16 per step), "
                   "a read-only copy of the decode kernel's loads on the c2 and c5 inputs (TB/s of their "
                   "algorithmic attention bytes)")
    torch.cuda.empty_cache()
    return res


def bench_bwd(torch, hip, steps, warmup):
    """Backward of a dense causal training shape through the C ABI
    (fa_mha_bwd): B=4, S=4096, H=32/8, D=128, bf16. Algorithmic FLOPs follow
    the usual FlashAttention count, 2.5 x the forward's 4*D per visible
    (query, key) pair (the five products S, dP, dV, dK, dQ at 2*D each); the
    kernels' recomputation of S and dP in the dQ pass is not counted."""
    from fa_mi355x import capi
    B, S, H, Hk, D = 4, 4096, 32, 8, 128
    gen = torch.Generator(device="cuda").manual_seed(6)
    rn = lambda *shape: torch.randn(shape, generator=gen, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    q, k, v, do = rn(B, S, H, D), rn(B, S, Hk, D), rn(B, S, Hk, D), rn(B, S, H, D)
    scale = D ** -0.5
    out, lse = torch.ops.fa_mi355x.fwd(q, k, v, None, 0.0, scale, True, -1, -1, 0.0)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    sd = torch.empty((B, H, S), device="cuda", dtype=torch.float32)
    kw = dict(dtype=capi.FA_DTYPE_BF16, batch=B, seqlen_q=S, seqlen_k=S, nheads=H, nheads_k=Hk, headdim=D,
              softmax_lse=lse.data_ptr(), softmax_d=sd.data_ptr(), softmax_scale=scale, is_causal=1)
    for n, t in (("q", q), ("k", k), ("v", v), ("out", out), ("dout", do), ("dq", dq), ("dk", dk), ("dv", dv)):
        kw.update({n: t.data_ptr(), f"{n}_batch_stride": t.stride(0), f"{n}_row_stride": t.stride(1),
                   f"{n}_head_stride": t.stride(2)})
    p = capi.new_bwd_params(**kw)
    stream = torch.cuda.current_stream().cuda_stream

    def call():
        if capi.backward(p, capi.FA_KIND_DENSE, stream) != 0:
            raise RuntimeError(capi.last_error())

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < WARM_MS * 1e-3:
        call()
        torch.cuda.synchronize()
    a, b = hip.event(), hip.event()
    hip.record(a, stream)
    for _ in range(steps):
        call()
    hip.record(b, stream)
    us = hip.ms(a, b) / steps * 1e3
    torch.cuda.synchronize()
    pairs = S * (S + 1) // 2
    flops = 2.5 * 4 * D * pairs * B * H
    return {"us_per_call": us, "flops_per_call": flops, "tflops_call": flops / (us * 1e-6) / 1e12,
            "frac_mfma": flops / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS,
            "workload": f"backward, dense causal B{B} S{S} H{H}/{Hk} D{D} bf16 (dQ with dsum, then dK/dV kernels)"}


TRAFFIC_PROFILES = ("profiles/fa_attention_kernels_hbm_traffic.txt", "profiles/fa_decode_kernel_fp8_hbm_traffic.txt")


def traffic_source(cfg):
    """The profile summary that holds `cfg`'s measured traffic, or None."""
    import re
    for rel in TRAFFIC_PROFILES:
        path = os.path.join(REPO, rel)
        if os.path.exists(path) and re.search(r"^traffic_bytes_per_launch\[%s\]\s*=" % cfg, open(path).read(), re.M):
            return rel
    return None


def measured_traffic(cfg):
    """HBM bytes per launch of the attention kernel on `cfg`, as measured by the two
    rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) summarised in TRAFFIC_PROFILES
    (scaled by the plain-copy calibration recorded there); None if absent."""
    import re
    rel = traffic_source(cfg)
    if rel is None:
        return None
    m = re.search(r"^traffic_bytes_per_launch\[%s\]\s*=\s*(\d+)" % cfg, open(os.path.join(REPO, rel)).read(), re.M)
    return int(m.group(1))


PHASES_LIB = os.path.join(REPO, "flash-attention-npu_amd", "fa_mi355x", "lib", "libfa_mi355x_phases.so")


def decode_phases(names, torch, hip, reps):
    """Phase breakdown of the decode kernel from the per-wave real-time stamps
    (100 MHz) of the instrumented library (build.py: FA_DECODE_PHASES), in µs,
    medians over `reps` calls:
      plan        entry -> end of the in-LDS plan (median wave)
      first_tile  end of the plan -> end of the wave's first tile (median wave)
      start       kernel start -> median first-tile end (plan + pipeline fill)
      steady      median first-tile end -> median wave exit
      tail        median wave exit -> last wave exit
      kernel      first wave entry -> last wave exit
      merge       the merge kernel (stage events around it)
    plus the median exit per XCD and per segment count."""
    import numpy as np
    from fa_mi355x import capi
    if not os.path.exists(PHASES_LIB):
        raise SystemExit(f"{PHASES_LIB} is not built: run python flash-attention-npu_amd/build.py --phases first")
    L = ctypes.CDLL(PHASES_LIB, mode=os.RTLD_LOCAL)
    L.fa_mha_fwd_kvcache.argtypes = [ctypes.POINTER(capi.FwdParams), ctypes.c_void_p]
    L.fa_decode_phase_stamps.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int)]
    hip.lib.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.lib.hipMemset.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
    stream = torch.cuda.current_stream().cuda_stream
    workers = torch.cuda.get_device_properties(0).multi_processor_count * 4
    out = {}
    for name in names:
        ncopy = {"c2": 2, "c3": 2, "c5": 4, "c2f8": 2, "c3f8": 2}[name]
        c = build_case(name, torch, "cuda", ncopy)
        ps = c["params"]
        buf, cap = ctypes.c_void_p(), ctypes.c_int()
        assert L.fa_decode_phase_stamps(ctypes.byref(buf), ctypes.byref(cap)) == 0
        assert workers <= cap.value
        for i in range(20):
            assert L.fa_mha_fwd_kvcache(ctypes.byref(ps[i % len(ps)]), stream) == 0
        torch.cuda.synchronize()
        runs = []
        for rep in range(reps):
            assert hip.lib.hipMemset(buf, 0, cap.value * 64) == 0
            p = ps[rep % len(ps)]
            evs = [hip.event() for _ in range(4)]
            arr = (ctypes.c_void_p * 4)(*[e.value for e in evs])
            p.stage_events = ctypes.cast(arr, ctypes.c_void_p)
            assert L.fa_mha_fwd_kvcache(ctypes.byref(p), stream) == 0
            p.stage_events = None
            torch.cuda.synchronize()
            merge_us = hip.ms(evs[2], evs[3]) * 1e3
            raw = np.zeros(cap.value * 8, dtype=np.uint64)
            assert hip.lib.hipMemcpy(raw.ctypes.data, buf, raw.nbytes, 2) == 0
            s = raw.reshape(cap.value, 8)[:workers].astype(np.int64)
            live = s[:, 5] > 0
            k0 = s[:, 0].min()
            us = lambda col: (col - k0) / 100.0  # 100 MHz ticks -> µs
            entry, plan, first, exit_ = us(s[:, 0]), us(s[:, 1]), us(s[:, 2]), us(s[:, 3])
            med_exit = float(np.median(exit_[live]))
            med_first = float(np.median(first[live]))
            xcc = s[:, 7] & 0xF
            r = {"plan": float(np.median(plan - entry)), "first_tile": float(np.median((first - plan)[live])),
                 "start": med_first, "steady": med_exit - med_first, "tail": float(exit_.max()) - med_exit,
                 "kernel": float(exit_.max()), "dispatch_spread": float(entry.max()),
                 "exit_p10": float(np.percentile(exit_[live], 10)), "exit_p90": float(np.percentile(exit_[live], 90)),
                 "merge": merge_us, "tiles_per_wave": float(s[live, 5].mean()),
                 "segments_mean": float(s[live, 4].mean()), "segments_max": int(s[live, 4].max())}
            # spread of the exits between CUs and within a CU (HW_ID: CU, SH, SE fields)
            hw = s[:, 6]
            cu = xcc * 1000 + ((hw >> 13) & 7) * 100 + ((hw >> 12) & 1) * 16 + ((hw >> 8) & 15)
            ids = np.unique(cu[live])
            means = np.array([exit_[live & (cu == u)].mean() for u in ids])
            within = np.concatenate([exit_[live & (cu == u)] - exit_[live & (cu == u)].mean() for u in ids])
            r["exit_sd_between_cu"] = float(means.std())
            r["exit_sd_within_cu"] = float(within.std())
            for x in range(8):
                sel = live & (xcc == x)
                r[f"exit_xcd{x}"] = float(np.median(exit_[sel])) if sel.any() else None
            for n in sorted(set(s[live, 4].tolist()))[:8]:
                sel = live & (s[:, 4] == n)
                r[f"exit_nseg{n}"] = float(np.median(exit_[sel]))
            runs.append(r)
        med = {}
        for k in runs[0]:
            vals = [rr[k] for rr in runs if rr.get(k) is not None]
            med[k] = round(float(np.median(vals)), 2) if vals else None
        med["workload"] = c["work_desc"]
        out[name] = med
        print(f"# {name}: {json.dumps(med)}", file=sys.stderr, flush=True)
        del c
        torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="c2,c3,c4,c5,bwd,c2f8,c3f8")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--ceilings", action="store_true",
                    help="also measure this part's practical HBM and bf16 GEMM ceilings with library kernels")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 3 plain device copies of 1 GiB (reference for rocprof FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--phases", action="store_true",
                    help="instead of the bench line: the decode kernel's per-wave phase breakdown on the decode "
                         "configs of --configs, from the instrumented library (libfa_mi355x_phases.so)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the per-GPU shard of the decode/prefill work is the single-GPU workload reported with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import fa_mi355x  # noqa: F401  (fails loudly without the built HIP library)
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = "cuda"
    hip = Hip()
    names = [s.strip() for s in args.configs.split(",") if s.strip()]
    if args.phases:
        dec = [n for n in names if n in ("c2", "c3", "c5", "c2f8", "c3f8")]
        print(json.dumps({"phases_us": decode_phases(dec, torch, hip, max(args.steps, 1))}))
        return
    if "c2" not in names:
        names = ["c2"] + names
    results = {}
    for name in names:
        if name == "bwd":
            r = bench_bwd(torch, hip, args.steps, args.warmup)
            results[name] = r
            print(f"# {name}: {json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()})}",
                  file=sys.stderr, flush=True)
            torch.cuda.empty_cache()
            continue
        ncopy = {"c2": 2, "c3": 2, "c4": 1, "c5": 4, "c2f8": 2, "c3f8": 2}[name]
        c = build_case(name, torch, dev, ncopy)
        torch.cuda.synchronize()
        t = time_case(c, hip, torch, args.steps, args.warmup)
        r = dict(t)
        r["workload"] = c["work_desc"]
        if name != "c4":
            # only c4 launches an append kernel (kv_prep); c2 / c3 / c2f8 / c3f8
            # append their one token inside the decode kernel and c5 appends
            # nothing, so their append stage times only the two event packets.
            # That figure is the event cost carried by attn_us and combine_us too.
            r["append_us"] = None
            r["event_pair_us"] = t["append_us"]
        if c["bound"] == "hbm":
            r["bytes_per_call"] = c["bytes"]
            r["tbps_call"] = c["bytes"] / (t["us_per_call"] * 1e-6) / 1e12
            r["attn_bytes"] = c["attn_bytes"]
            r["attn_tbps"] = c["attn_bytes"] / (t["attn_us"] * 1e-6) / 1e12
            r["attn_frac_hbm"] = r["attn_tbps"] * 1e3 / HBM_PEAK_GBS
            r["roofline"] = {"bound": "hbm", "achieved": round(r["attn_tbps"] * 1e3, 1), "peak": HBM_PEAK_GBS,
                             "unit": "GB/s", "frac": round(r["attn_frac_hbm"], 4),
                             "traffic": measured_traffic(name), "traffic_source": traffic_source(name),
                             "kernel": "fa_decode_kernel",
                             "kernel_us": round(t["attn_us"], 2), "algorithmic_bytes": c["attn_bytes"]}
        else:
            r["flops_per_call"] = c["flops"]
            r["tflops_call"] = c["flops"] / (t["us_per_call"] * 1e-6) / 1e12
            r["attn_tflops"] = c["flops"] / (t["attn_us"] * 1e-6) / 1e12
            r["attn_frac_mfma"] = r["attn_tflops"] / BF16_PEAK_TFLOPS
            r["roofline"] = {"bound": "mfma", "achieved": round(r["attn_tflops"], 1), "peak": BF16_PEAK_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(r["attn_frac_mfma"], 4), "traffic": measured_traffic(name),
                             "kernel": "fa_prefill_kernel", "kernel_us": round(t["attn_us"], 2),
                             "algorithmic_flops": c["flops"]}
        if not args.no_cpu and name in ("c2", "c3", "c4", "c5"):
            r["cpu_baseline"], ref = cpu_baseline(c, torch)
            r["parity"] = parity(c, ref, torch)
        results[name] = r
        print(f"# {name}: {json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()})}",
              file=sys.stderr, flush=True)
        del c
        torch.cuda.empty_cache()

    if args.copy_calibration:
        src = torch.ones(1 << 28, dtype=torch.int32, device=dev)  # 1 GiB read, 1 GiB written
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    c2 = results["c2"]
    traffic = measured_traffic("c2")
    traffic_src = traffic_source("c2")
    cpu = c2.get("cpu_baseline")
    if args.ceilings:
        results["ceilings"] = ceilings(torch, hip)
        print(f"# ceilings: {json.dumps(results['ceilings'])}", file=sys.stderr, flush=True)
    line = {
        "metric": METRIC,
        "value": round(c2["tbps_call"], 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c2["us_per_call"] / 1e3, 6),
        "us_per_call": round(c2["us_per_call"], 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1))",
        "config": {"workload": "BASELINE config 2: " + c2["workload"], "batch": 32, "nheads": 32, "nheads_k": 8,
                   "headdim": 128, "seqlen_cache": 8192, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(c2["attn_tbps"] * 1e3, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(c2["attn_frac_hbm"], 4), "traffic": traffic,
                     "kernel": "fa_decode_kernel", "kernel_us": round(c2["attn_us"], 2),
                     "algorithmic_bytes": c2["attn_bytes"],
                     "traffic_source": traffic_src},
        "cpu_baseline": cpu,
        "parity": c2.get("parity"),
        "configs": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in results.items()},
        "host_cores": os.cpu_count(),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
