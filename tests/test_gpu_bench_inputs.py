"""Parity on the benchmarked inputs themselves: BASELINE configs 2, 3 and 5
built by bench.py's own seeded builder (build_case), one call through the C
ABI (as bench.py makes it), and every sequence and head checked against the
oracle: out max-abs within 1e-2 (bf16), LSE within 1e-4 relative, and the
caches after the one-token append bit for bit (configs 2 and 3; config 5
appends nothing). Config 4 at full size is tests/test_gpu_regimes.py."""
import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import fa_oracle as orc
from tests._util import assert_close_lse, assert_close_out, bits

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


@pytest.mark.parametrize("name", ["c2", "c3", "c5"])
def test_benchmarked_inputs_full(name):
    import bench
    from fa_mi355x import capi
    print(f"case bench inputs {name}: every sequence against the oracle", flush=True)
    c = bench.build_case(name, torch, "cuda", 1)
    q, kn, vn, caches, bt, bidx, cos, sin, alibi, out, lse, sl = c["keep"]
    kc, vc = caches[0]
    kh, vh = bits(kc), bits(vc)  # the caches before the call
    p = c["params"][0]
    st = capi.lib().fa_mha_fwd_kvcache(ctypes.byref(p), torch.cuda.current_stream().cuda_stream)
    assert st == capi.FA_OK, capi.last_error()
    torch.cuda.synchronize()
    ro, rl, rk, rv = orc.kvcache_forward(
        bits(q), kh, vh, dtype=orc.BF16, cache_seqlens=c["L"].numpy(), k=None if kn is None else bits(kn),
        v=None if vn is None else bits(vn), block_table=None if bt is None else bt.cpu().numpy(),
        cache_batch_idx=None if bidx is None else bidx.cpu().numpy(), causal=True,
        window=(4096, 0) if name == "c5" else (-1, -1), alibi=None if alibi is None else alibi.cpu().numpy(),
        nthreads=NT)
    if kn is not None:
        assert np.array_equal(bits(kc), rk), "k_cache after the append is not bit-exact"
        assert np.array_equal(bits(vc), rv), "v_cache after the append is not bit-exact"
    else:
        assert np.array_equal(bits(kc), kh) and np.array_equal(bits(vc), vh), "the caches changed"
    mx = assert_close_out(out, ro, torch.bfloat16)
    rel = assert_close_lse(lse, rl)
    print(f"  {name}: {c['B']} sequences, out max-abs {mx:.2e}, lse rel {rel:.1e}", flush=True)
