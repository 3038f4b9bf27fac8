"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from an fp64 brute force, not from the oracle)
against the CPU oracle and, on a GPU, against the HIP path through the public
flash_attn_npu_v2 / v3 APIs. Bars: out max-abs 2e-3 (fp16) / 1e-2 (bf16),
LSE 1e-4 relative, appended caches bit-exact."""
import glob
import json
import os

import numpy as np
import pytest
import torch

from oracle import fa_oracle as orc
from tests._util import LSE_ATOL, LSE_RTOL

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FILES = sorted(glob.glob(os.path.join(GOLDEN, "*.npz")))
NAMES = [os.path.basename(f)[:-4] for f in FILES]
TOL = {"fp16": 2e-3, "bf16": 1e-2}
ODT = {"fp16": orc.FP16, "bf16": orc.BF16}
TDT = {"fp16": torch.float16, "bf16": torch.bfloat16}


def load(name):
    z = np.load(os.path.join(GOLDEN, name + ".npz"))  # allow_pickle stays False
    d = {k: z[k] for k in z.files}
    d["meta"] = json.loads(str(d["meta"]))
    return d


def check(out_f32, lse, d):
    m = d["meta"]
    err = np.abs(out_f32.reshape(d["out"].shape) - d["out"])
    assert err.max() <= TOL[m["dtype"]], f"out max-abs {err.max():.3e}"
    ref = d["lse"]
    lse = np.asarray(lse, np.float32).reshape(ref.shape)
    inf = np.isinf(ref)
    assert np.array_equal(np.isinf(lse), inf), "empty-row (+inf) pattern differs"
    if (~inf).any():
        err = np.abs(lse[~inf].astype(np.float64) - ref[~inf])
        assert (err <= LSE_RTOL * np.abs(ref[~inf]) + LSE_ATOL).all(), f"LSE off by {err.max():.3e}"


def test_fixtures_present():
    assert len(NAMES) >= 8, NAMES


@pytest.mark.parametrize("name", NAMES)
def test_oracle_matches_golden(name):
    d = load(name)
    m = d["meta"]
    dt = ODT[m["dtype"]]
    w = tuple(m["window"])
    if m["kind"] == "dense":
        out, lse = orc.attention(d["q"], d["k"], d["v"], dtype=dt, scale=m["scale"], causal=m["causal"], window=w,
                                 softcap=m["softcap"], alibi=d.get("alibi"), nthreads=4)
    elif m["kind"] == "varlen":
        out, lse = orc.attention(d["q"], d["k"], d["v"], dtype=dt, scale=m["scale"], causal=m["causal"], window=w,
                                 cu_seqlens_q=d["cu_seqlens_q"], cu_seqlens_k=d["cu_seqlens_k"],
                                 max_seqlen_q=m["max_seqlen_q"], nthreads=4)
    else:
        rot = m["rotary"]
        out, lse, kc, vc = orc.kvcache_forward(
            d["q"], d["k_cache"], d["v_cache"], dtype=dt, cache_seqlens=d["cache_seqlens"], k=d.get("k"),
            v=d.get("v"), rotary_cos=d.get("rotary_cos"), rotary_sin=d.get("rotary_sin"),
            rotary_interleaved=bool(rot and rot["interleaved"]), cache_batch_idx=d.get("cache_batch_idx"),
            block_table=d.get("block_table"), softmax_scale=m["scale"], causal=m["causal"], window=w,
            alibi=d.get("alibi"), nthreads=4)
        if m["s_new"]:
            assert np.array_equal(kc, d["k_cache_after"]) and np.array_equal(vc, d["v_cache_after"])
    check(orc.from_bits(out, dt).reshape(out.shape), lse, d)


def _t(a, dt=None):
    """numpy -> cuda tensor (16-bit patterns reinterpreted as dtype `dt`)."""
    if a is None:
        return None
    if dt is not None:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dt).cuda()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("api", ["v2", "v3"])
@pytest.mark.parametrize("name", NAMES)
def test_hip_matches_golden(name, api):
    import flash_attn_npu_v2 as v2
    import flash_attn_npu_v3 as v3
    print(f"case golden {name} {api}", flush=True)
    d = load(name)
    m = d["meta"]
    tdt = TDT[m["dtype"]]
    w = tuple(m["window"])
    al = _t(d.get("alibi"))
    if m["kind"] == "dense":
        if api == "v3" and al is not None:
            pytest.skip("the v3 flash_attn_func has no alibi argument")
        q, k, v = _t(d["q"], tdt), _t(d["k"], tdt), _t(d["v"], tdt)
        if api == "v2":
            out, lse, _ = v2.flash_attn_func(q, k, v, softmax_scale=m["scale"], causal=m["causal"], window_size=w,
                                             softcap=m["softcap"], alibi_slopes=al, return_attn_probs=True)
        else:
            out, lse = v3.flash_attn_func(q, k, v, softmax_scale=m["scale"], causal=m["causal"], window_size=w,
                                          softcap=m["softcap"], return_attn_probs=True)
    elif m["kind"] == "varlen":
        q, k, v = _t(d["q"], tdt), _t(d["k"], tdt), _t(d["v"], tdt)
        cq, ck = _t(d["cu_seqlens_q"]), _t(d["cu_seqlens_k"])
        f = v2.flash_attn_varlen_func if api == "v2" else v3.flash_attn_varlen_func
        res = f(q, k, v, cq, ck, m["max_seqlen_q"], m["max_seqlen_k"], softmax_scale=m["scale"], causal=m["causal"],
                window_size=w, return_attn_probs=True)
        out, lse = res[0], res[1]
    else:
        if api == "v3" and al is not None:
            pytest.skip("the v3 flash_attn_with_kvcache has no alibi argument")
        rot = m["rotary"]
        kc, vc = _t(d["k_cache"], tdt), _t(d["v_cache"], tdt)
        kw = dict(k=_t(d.get("k"), tdt), v=_t(d.get("v"), tdt), rotary_cos=_t(d.get("rotary_cos"), tdt),
                  rotary_sin=_t(d.get("rotary_sin"), tdt), cache_seqlens=_t(d["cache_seqlens"]),
                  cache_batch_idx=_t(d.get("cache_batch_idx")), softmax_scale=m["scale"], causal=m["causal"],
                  window_size=w, rotary_interleaved=bool(rot and rot["interleaved"]), return_softmax_lse=True)
        if api == "v2":
            out, lse = v2.flash_attn_with_kvcache(_t(d["q"], tdt), kc, vc, block_table=_t(d.get("block_table")),
                                                  alibi_slopes=al, **kw)
        else:
            out, lse, *_ = v3.flash_attn_with_kvcache(_t(d["q"], tdt), kc, vc, page_table=_t(d.get("block_table")),
                                                      **kw)
        torch.cuda.synchronize()
        if m["s_new"]:
            got_k = kc.cpu().view(torch.int16).numpy().view(np.uint16)
            got_v = vc.cpu().view(torch.int16).numpy().view(np.uint16)
            assert np.array_equal(got_k, d["k_cache_after"]), "k_cache append is not bit-exact"
            assert np.array_equal(got_v, d["v_cache_after"]), "v_cache append is not bit-exact"
    torch.cuda.synchronize()
    check(out.float().cpu().numpy(), lse.float().cpu().numpy(), d)
