"""GPU parity of the v3 kvcache extensions and attention_chunk: the HIP path
(flash_attn_npu_v3 -> torch op -> C ABI) against the CPU oracle
(oracle.fa_oracle.kvcache_forward_v3 / attention with chunk) on identical
seeded inputs. Tolerances as everywhere: out max-abs 2e-3 (fp16) / 1e-2 (bf16)
plus one ulp of the reference value, LSE 1e-4 relative, the cache after
the append bit-exact."""
import os

import numpy as np
import pytest
import torch

from oracle import fa_oracle as orc
from tests._util import assert_close_lse, assert_close_out, bits, odt, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
NT = min(16, os.cpu_count() or 1)


def _rope(n, rd, dtype):
    inv = 1.0 / (10000.0 ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd))
    ang = torch.arange(n, dtype=torch.float32)[:, None] * inv[None, :]
    return torch.cos(ang).to(dtype), torch.sin(ang).to(dtype)


def run_v3(*, H=32, Hk=8, D=128, dtype=torch.bfloat16, q_lens, new_lens, seqlens, capacity=0, page=0,
           ragged_q=False, ragged_new=False, leftpad=None, rotary=None, rot_dim=None, rotary_seqlens=None,
           causal=True, window=(-1, -1), chunk=0, num_splits=0, seed=0):
    """q_lens / new_lens: per-sequence query / new-token counts (all equal when
    the layout is dense); seqlens: cached tokens; leftpad: first valid slot."""
    import flash_attn_npu_v3
    print(f"case v3kv q={q_lens} new={new_lens} L={seqlens} page={page} lp={leftpad} rot={rotary} chunk={chunk}",
          flush=True)
    g = torch.Generator().manual_seed(seed)
    B = len(q_lens)
    L = np.asarray(seqlens, np.int32)
    if ragged_q:
        q = randn((sum(q_lens), H, D), dtype, g, "cpu")
        cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    else:
        assert len(set(q_lens)) == 1
        q = randn((B, q_lens[0], H, D), dtype, g, "cpu")
        cu_q = None
    kn = vn = None
    cu_n = None
    if max(new_lens) > 0:
        if ragged_new:
            kn = randn((sum(new_lens), Hk, D), dtype, g, "cpu")
            vn = randn((sum(new_lens), Hk, D), dtype, g, "cpu")
            cu_n = np.concatenate([[0], np.cumsum(new_lens)]).astype(np.int32)
        else:
            assert len(set(new_lens)) == 1
            kn = randn((B, new_lens[0], Hk, D), dtype, g, "cpu")
            vn = randn((B, new_lens[0], Hk, D), dtype, g, "cpu")
    bt = None
    if page:
        need = [(int(L[b]) + new_lens[b] + page - 1) // page for b in range(B)]
        mb = max(max(need), 1)
        nblocks = sum(need) + 3
        perm = torch.randperm(nblocks, generator=g).to(torch.int32)
        bt = torch.zeros((B, mb), dtype=torch.int32)
        o = 0
        for b in range(B):
            bt[b, :need[b]] = perm[o:o + need[b]]
            o += need[b]
        kc = randn((nblocks, page, Hk, D), dtype, g, "cpu")
        vc = randn((nblocks, page, Hk, D), dtype, g, "cpu")
    else:
        kc = randn((B, capacity, Hk, D), dtype, g, "cpu")
        vc = randn((B, capacity, Hk, D), dtype, g, "cpu")
    cos = sin = None
    if rotary:
        n = int(L.max()) + max(new_lens) + max(q_lens)
        if rotary_seqlens is not None:
            n = max(n, int(np.max(rotary_seqlens)) + max(new_lens) + max(q_lens))
        cos, sin = _rope(n + 8, rot_dim or D, dtype)
    inter = rotary == "interleaved"
    # oracle first (host copies)
    ro, rl, rk, rv = orc.kvcache_forward_v3(
        bits(q), bits(kc), bits(vc), dtype=odt(dtype), cache_seqlens=L,
        k=None if kn is None else bits(kn), v=None if vn is None else bits(vn),
        rotary_cos=None if cos is None else bits(cos), rotary_sin=None if sin is None else bits(sin),
        rotary_interleaved=inter, block_table=None if bt is None else bt.numpy(), causal=causal, window=window,
        cache_leftpad=leftpad, rotary_seqlens=rotary_seqlens, cu_seqlens_q=cu_q,
        max_seqlen_q=max(q_lens), cu_seqlens_k_new=cu_n, attention_chunk=chunk, nthreads=NT)
    t = lambda a: None if a is None else torch.as_tensor(np.asarray(a, np.int32)).to(DEV)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    out, lse, *_ = flash_attn_npu_v3.flash_attn_with_kvcache(
        q.to(DEV), kc_d, vc_d, k=None if kn is None else kn.to(DEV), v=None if vn is None else vn.to(DEV),
        rotary_cos=None if cos is None else cos.to(DEV), rotary_sin=None if sin is None else sin.to(DEV),
        cache_seqlens=t(L), cache_leftpad=t(leftpad), page_table=None if bt is None else bt.to(DEV),
        cu_seqlens_q=t(cu_q), cu_seqlens_k_new=t(cu_n), max_seqlen_q=max(q_lens) if ragged_q else None,
        rotary_seqlens=t(rotary_seqlens), causal=causal, window_size=window, attention_chunk=chunk,
        rotary_interleaved=inter, num_splits=num_splits, return_softmax_lse=True)
    torch.cuda.synchronize()
    assert np.array_equal(bits(kc_d), rk), "k_cache after the append differs"
    assert np.array_equal(bits(vc_d), rv), "v_cache after the append differs"
    assert_close_out(out, ro, dtype)
    assert_close_lse(lse, rl)


# ---- cache_leftpad ----------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_leftpad_fused_append(dtype):
    rng = np.random.default_rng(1)
    L = rng.integers(300, 2000, 6)
    run_v3(dtype=dtype, q_lens=[1] * 6, new_lens=[1] * 6, seqlens=L, capacity=2048,
           leftpad=rng.integers(0, 290, 6), seed=1)


def test_decode_leftpad_rotary_at_rotary_seqlens():
    rng = np.random.default_rng(2)
    L = rng.integers(100, 900, 4)
    run_v3(q_lens=[2] * 4, new_lens=[2] * 4, seqlens=L, capacity=1024, leftpad=rng.integers(0, 99, 4),
           rotary="neox", rotary_seqlens=rng.integers(0, 500, 4), seed=2)


@pytest.mark.parametrize("rotary", ["neox", "interleaved"])
def test_prefill_leftpad_rotary_chunk(rotary):
    rng = np.random.default_rng(3)
    L = rng.integers(200, 700, 3)
    run_v3(q_lens=[96] * 3, new_lens=[96] * 3, seqlens=L, capacity=1024, leftpad=rng.integers(0, 199, 3),
           rotary=rotary, rotary_seqlens=rng.integers(0, 400, 3), chunk=128, seed=3)


def test_leftpad_equal_to_seqlens():
    L = np.array([40, 700, 5])
    run_v3(q_lens=[1] * 3, new_lens=[1] * 3, seqlens=L, capacity=1024, leftpad=L, seed=4)


# ---- ragged q / ragged new tokens -----------------------------------------------------------------

def test_ragged_decode_paged():
    """Decode-sized ragged batch (1..4 queries, 0..3 new tokens per sequence) on a paged cache."""
    rng = np.random.default_rng(5)
    q_lens = [1, 4, 2, 1, 3]
    new_lens = [1, 3, 0, 1, 2]
    run_v3(q_lens=q_lens, new_lens=new_lens, seqlens=rng.integers(50, 1500, 5), page=256, ragged_q=True,
           ragged_new=True, seed=5)


@pytest.mark.parametrize("page", [0, 64])
def test_ragged_mixed_prefill_decode(page):
    """A serving batch: new prompts and decode steps together (queries = new tokens)."""
    q_lens = [1, 37, 1, 130, 5]
    run_v3(q_lens=q_lens, new_lens=q_lens, seqlens=[900, 0, 33, 200, 1400], capacity=2048, page=page,
           ragged_q=True, ragged_new=True, rotary="interleaved", seed=6)


def test_ragged_q_dense_new_rotary_seqlens_window():
    run_v3(q_lens=[3, 9, 1], new_lens=[4, 4, 4], seqlens=[10, 300, 77], capacity=512, ragged_q=True,
           rotary="neox", rot_dim=64, rotary_seqlens=[100, 7, 0], window=(50, 0), seed=7)


# ---- attention_chunk --------------------------------------------------------------------------------

@pytest.mark.parametrize("chunk", [32, 100, 512])
def test_decode_chunk(chunk):
    rng = np.random.default_rng(8)
    run_v3(q_lens=[3] * 4, new_lens=[1] * 4, seqlens=rng.integers(10, 3000, 4), page=128, chunk=chunk, seed=8)


def test_decode_chunk_split_and_headdim_64():
    run_v3(D=64, q_lens=[1], new_lens=[1], seqlens=[7000], capacity=8192, chunk=1000, num_splits=4, seed=9)


def test_prefill_chunk_headdim_256_leftpad():
    run_v3(H=8, Hk=2, D=256, q_lens=[70] * 2, new_lens=[70] * 2, seqlens=[90, 300], capacity=512,
           leftpad=[20, 0], chunk=64, seed=10)


def _dense_chunk(B, Sq, Sk, H, Hk, D, dtype, causal, window, chunk, seed, varlen=False):
    import flash_attn_npu_v3
    print(f"case chunk B={B} Sq={Sq} Sk={Sk} D={D} causal={causal} window={window} chunk={chunk}", flush=True)
    g = torch.Generator().manual_seed(seed)
    q = randn((B, Sq, H, D), dtype, g, "cpu")
    k = randn((B, Sk, Hk, D), dtype, g, "cpu")
    v = randn((B, Sk, Hk, D), dtype, g, "cpu")
    ro, rl = orc.attention(bits(q), bits(k), bits(v), dtype=odt(dtype), scale=D ** -0.5, causal=causal,
                           window=window, nthreads=NT, chunk=chunk)
    if varlen:
        cu_q = torch.arange(B + 1, dtype=torch.int32) * Sq
        cu_k = torch.arange(B + 1, dtype=torch.int32) * Sk
        out, lse = flash_attn_npu_v3.flash_attn_varlen_func(
            q.reshape(B * Sq, H, D).to(DEV), k.reshape(B * Sk, Hk, D).to(DEV), v.reshape(B * Sk, Hk, D).to(DEV),
            cu_q.to(DEV), cu_k.to(DEV), Sq, Sk, causal=causal, window_size=window, attention_chunk=chunk,
            return_attn_probs=True)
        out = out.reshape(B, Sq, H, D)
        lse = lse.reshape(H, B, Sq).permute(1, 0, 2)
    else:
        out, lse = flash_attn_npu_v3.flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal,
                                                     window_size=window, attention_chunk=chunk,
                                                     return_attn_probs=True)
    torch.cuda.synchronize()
    assert_close_out(out, ro, dtype)
    assert_close_lse(lse, rl)


@pytest.mark.parametrize("case", [
    (2, 500, 500, 8, 2, 128, torch.bfloat16, True, (-1, -1), 64),
    (2, 300, 700, 8, 8, 128, torch.float16, False, (-1, -1), 100),
    (1, 257, 257, 4, 1, 64, torch.bfloat16, True, (40, 0), 96),
    (2, 200, 150, 4, 2, 256, torch.bfloat16, True, (-1, -1), 32),   # Sq > Sk
    (1, 64, 4000, 8, 2, 128, torch.bfloat16, True, (-1, -1), 1024),  # few rows: split over the keys
])
def test_dense_chunk(case):
    _dense_chunk(*case, seed=11)


def test_varlen_chunk():
    _dense_chunk(3, 130, 130, 8, 2, 128, torch.bfloat16, True, (-1, -1), 48, seed=12, varlen=True)


# ---- head dims that are not a multiple of 8 (the v3 API runs them zero-padded) --------------------

@pytest.mark.parametrize("D,page", [(111, 0), (111, 64), (36, 0)])
def test_unaligned_headdim_decode_append(D, page):
    rng = np.random.default_rng(600 + D + page)
    run_v3(H=16, Hk=4, D=D, q_lens=[1] * 4, new_lens=[1] * 4, seqlens=rng.integers(20, 1900, 4), capacity=2048,
           page=page, seed=600 + D + page)


def test_unaligned_headdim_prefill_rotary_window():
    rng = np.random.default_rng(610)
    run_v3(H=8, Hk=2, D=111, q_lens=[70] * 3, new_lens=[70] * 3, seqlens=rng.integers(100, 900, 3), capacity=1024,
           rotary="neox", rot_dim=96, window=(200, 0), seed=610)
