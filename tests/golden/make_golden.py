"""Writes the golden fixtures tests/golden/*.npz (run: python tests/golden/make_golden.py).

The reference ships no vectors for this path (its tests draw unseeded random
inputs at run time), so the fixtures are made here, from fixed seeds, without
the C oracle: the expected outputs come from the float64 brute force in
brute.py, the expected caches from numpy indexing, and the rotated keys from
numpy float32 arithmetic (each product and sum rounded separately, as the
reference docstring's fp32 rotary is: x1*cos - x2*sin, x2*cos + x1*sin) with
round-to-nearest-even into the 16-bit dtype by torch.

Each file holds the inputs as raw 16-bit patterns (uint16), int32 index
arrays, fp32 slopes / cos / sin, a `meta` JSON string (shapes, flags, dtype),
and the expected `out` (fp32 of the fp64 result), `lse` (fp32) and, when
tokens are appended, the caches after the append (uint16).
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import brute  # noqa: E402

TDT = {"fp16": torch.float16, "bf16": torch.bfloat16}


def to16(x, dt):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(TDT[dt]).view(torch.int16).numpy().view(
        np.uint16)


def from16(b, dt):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(TDT[dt]).float().numpy()


def rnd(rng, shape, dt):
    return to16(rng.standard_normal(shape).astype(np.float32), dt)


def rope(x16, cos16, sin16, pos, dt, interleaved):
    """x16 (S, H, D) bits rotated at positions pos (S,), cos/sin (N, rd/2) bits."""
    x = from16(x16, dt)
    c = from16(cos16, dt)[pos][:, None, :]
    s = from16(sin16, dt)[pos][:, None, :]
    rd = 2 * cos16.shape[1]
    y = x.copy()
    if interleaved:
        x1, x2 = x[..., 0:rd:2], x[..., 1:rd:2]
    else:
        x1, x2 = x[..., :rd // 2], x[..., rd // 2:rd]
    a = np.float32(x1 * c)
    b = np.float32(x2 * s)
    o1 = np.float32(a - b)
    o2 = np.float32(np.float32(x2 * c) + np.float32(x1 * s))
    if interleaved:
        y[..., 0:rd:2], y[..., 1:rd:2] = o1, o2
    else:
        y[..., :rd // 2], y[..., rd // 2:rd] = o1, o2
    return to16(y, dt)


def rope_tables(n, rd, dt):
    inv = 1.0 / 10000.0 ** (np.arange(0, rd, 2, dtype=np.float64) / rd)
    ang = np.outer(np.arange(n), inv)
    return to16(np.cos(ang), dt), to16(np.sin(ang), dt)


def save(name, meta, **arrays):
    np.savez_compressed(os.path.join(HERE, name + ".npz"), meta=np.array(json.dumps(meta)), **arrays)
    print("wrote", name, {k: v.shape for k, v in arrays.items()})


def dense_c1_small():
    """BASELINE config 1 reduced to one sequence of 256: dense causal fp16."""
    dt, B, S, H, D = "fp16", 1, 256, 2, 128
    rng = np.random.default_rng(101)
    q, k, v = (rnd(rng, (B, S, H, D), dt) for _ in range(3))
    scale = D ** -0.5
    out, lse = brute.attention_batch(from16(q, dt), from16(k, dt), from16(v, dt), [S] * B, scale, causal=True)
    save("dense_c1_small", dict(kind="dense", dtype=dt, causal=True, window=[-1, -1], softcap=0.0, scale=scale),
         q=q, k=k, v=v, out=out.astype(np.float32), lse=lse.astype(np.float32))


def dense_window_softcap_alibi():
    dt, B, Sq, Sk, H, Hk, D = "bf16", 2, 64, 128, 4, 2, 128
    rng = np.random.default_rng(102)
    q = rnd(rng, (B, Sq, H, D), dt)
    k, v = rnd(rng, (B, Sk, Hk, D), dt), rnd(rng, (B, Sk, Hk, D), dt)
    slopes = (2.0 ** (-8.0 * (np.arange(H) + 1) / H)).astype(np.float32)
    scale, window, cap = D ** -0.5, (48, 8), 10.0
    out, lse = brute.attention_batch(from16(q, dt), from16(k, dt), from16(v, dt), [Sk] * B, scale, False, window,
                                     slopes, cap)
    save("dense_window_softcap_alibi", dict(kind="dense", dtype=dt, causal=False, window=list(window), softcap=cap,
                                            scale=scale), q=q, k=k, v=v, alibi=slopes, out=out.astype(np.float32),
         lse=lse.astype(np.float32))


def varlen_gqa():
    dt, H, Hk, D = "fp16", 6, 2, 128
    rng = np.random.default_rng(103)
    lq, lk = [17, 1, 40], [17, 300, 25]
    cu_q = np.cumsum([0] + lq).astype(np.int32)
    cu_k = np.cumsum([0] + lk).astype(np.int32)
    q = rnd(rng, (cu_q[-1], H, D), dt)
    k, v = rnd(rng, (cu_k[-1], Hk, D), dt), rnd(rng, (cu_k[-1], Hk, D), dt)
    scale = 0.1
    out = np.zeros(q.shape, np.float64)
    lse = np.zeros((H, cu_q[-1]))
    for b in range(3):
        qs, ks = slice(cu_q[b], cu_q[b + 1]), slice(cu_k[b], cu_k[b + 1])
        o, l = brute.attention(from16(q[qs], dt), from16(k[ks], dt), from16(v[ks], dt), scale, causal=True)
        out[qs], lse[:, qs] = o, l
    save("varlen_gqa", dict(kind="varlen", dtype=dt, causal=True, window=[-1, -1], softcap=0.0, scale=scale,
                            max_seqlen_q=max(lq), max_seqlen_k=max(lk)),
         q=q, k=k, v=v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, out=out.astype(np.float32), lse=lse.astype(np.float32))


def kvcache_case(name, seed, dt, B, Sq, H, Hk, seqlens, s_new, page=0, cap=0, batch_idx=None, rotary=None,
                 causal=True, window=(-1, -1), alibi=False, nblocks_extra=3):
    D = 128
    rng = np.random.default_rng(seed)
    seqlens = np.asarray(seqlens, np.int32)
    q = rnd(rng, (B, Sq, H, D), dt)
    rows = B if batch_idx is None else int(max(batch_idx)) + 1
    row_of = np.arange(B) if batch_idx is None else np.asarray(batch_idx, np.int32)
    arrays = {}
    if page:
        need = np.zeros(rows, int)
        for b in range(B):
            need[row_of[b]] = (seqlens[b] + s_new + page - 1) // page
        nb = int(need.sum()) + nblocks_extra
        perm = rng.permutation(nb).astype(np.int32)
        bt = np.zeros((rows, int(need.max())), np.int32)
        o = 0
        for r in range(rows):
            bt[r, :need[r]] = perm[o:o + need[r]]
            o += need[r]
        kc, vc = rnd(rng, (nb, page, Hk, D), dt), rnd(rng, (nb, page, Hk, D), dt)
        arrays["block_table"] = bt

        def slot(b, j):
            return bt[row_of[b], j // page], j % page
    else:
        kc, vc = rnd(rng, (rows, cap, Hk, D), dt), rnd(rng, (rows, cap, Hk, D), dt)

        def slot(b, j):
            return row_of[b], j
    kn = vn = None
    cos = sin = None
    kc2, vc2 = kc.copy(), vc.copy()
    qr = q
    if s_new:
        kn, vn = rnd(rng, (B, s_new, Hk, D), dt), rnd(rng, (B, s_new, Hk, D), dt)
        kins = kn
        if rotary:
            cos, sin = rope_tables(int(seqlens.max()) + s_new + 8, rotary["rd"], dt)
            il = rotary["interleaved"]
            kins = np.stack([rope(kn[b], cos, sin, seqlens[b] + np.arange(s_new), dt, il) for b in range(B)])
            same = not (causal or window[0] >= 0 or window[1] >= 0)
            qr = np.stack([rope(q[b], cos, sin, seqlens[b] + (0 if same else 1) * np.arange(Sq), dt, il)
                           for b in range(B)])
        for b in range(B):
            for t in range(s_new):
                blk, j = slot(b, seqlens[b] + t)
                kc2[blk, j] = kins[b, t]
                vc2[blk, j] = vn[b, t]
    slopes = (2.0 ** (-8.0 * (np.arange(H) + 1) / H)).astype(np.float32) if alibi else None
    scale = D ** -0.5
    total = seqlens + s_new
    # gather each sequence's keys from the (appended) cache by numpy indexing
    outs, lses = [], []
    for b in range(B):
        n = int(total[b])
        idx = [slot(b, j) for j in range(n)]
        kb = np.stack([kc2[i, j] for i, j in idx]) if n else np.zeros((0, Hk, D), np.uint16)
        vb = np.stack([vc2[i, j] for i, j in idx]) if n else np.zeros((0, Hk, D), np.uint16)
        o, l = brute.attention(from16(qr[b], dt), from16(kb, dt), from16(vb, dt), scale, causal, window, slopes)
        outs.append(o)
        lses.append(l)
    meta = dict(kind="kvcache", dtype=dt, causal=causal, window=list(window), softcap=0.0, scale=scale,
                page=page, s_new=s_new, rotary=rotary)
    arrays.update(q=q, k_cache=kc, v_cache=vc, cache_seqlens=seqlens, out=np.stack(outs).astype(np.float32),
                  lse=np.stack(lses).astype(np.float32))
    if batch_idx is not None:
        arrays["cache_batch_idx"] = np.asarray(batch_idx, np.int32)
    if s_new:
        arrays.update(k=kn, v=vn, k_cache_after=kc2, v_cache_after=vc2)
    if rotary:
        arrays.update(rotary_cos=cos, rotary_sin=sin)
    if alibi:
        arrays["alibi"] = slopes
    save(name, meta, **arrays)


def main():
    dense_c1_small()
    dense_window_softcap_alibi()
    varlen_gqa()
    # BASELINE config 2 in miniature: contiguous GQA decode + 1-token append
    kvcache_case("decode_contiguous_append", 201, "bf16", B=3, Sq=1, H=8, Hk=2, seqlens=[0, 77, 126], s_new=1,
                 cap=128)
    # config 3 in miniature: paged (page 16) decode, permuted blocks, append
    kvcache_case("decode_paged_append", 202, "bf16", B=3, Sq=1, H=8, Hk=1, seqlens=[15, 16, 200], s_new=1, page=16)
    # config 4 in miniature: chunked prefill with NeoX rotary onto a cache
    kvcache_case("prefill_rotary_neox", 203, "bf16", B=2, Sq=24, H=4, Hk=2, seqlens=[40, 7], s_new=24, cap=96,
                 rotary=dict(rd=128, interleaved=False))
    kvcache_case("prefill_rotary_interleaved_partial", 204, "fp16", B=1, Sq=5, H=4, Hk=4, seqlens=[30], s_new=5,
                 cap=48, rotary=dict(rd=64, interleaved=True))
    # config 5 in miniature: spec-verify, paged, cache_batch_idx, window + ALiBi, no append
    kvcache_case("verify_window_alibi_paged", 205, "bf16", B=3, Sq=4, H=4, Hk=1, seqlens=[200, 90, 300], s_new=0,
                 page=32, batch_idx=[2, 0, 3], window=(64, 0), alibi=True)


if __name__ == "__main__":
    main()
