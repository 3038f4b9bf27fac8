"""Host-side checks of the C ABI (include/fa_mi355x.h) and the torch operator
layer, with no GPU: the library loads and exports every declared entry point,
the ctypes mirror of fa_fwd_params has the C layout, fa_validate rejects bad
arguments with the reference's messages, the operators have meta shapes, and
nothing falls back to a CPU path."""
import ctypes
import os
import re
import subprocess
import sys

import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "fa_mi355x.h")
PKG = os.path.join(REPO, "flash-attention-npu_amd")


@pytest.fixture(scope="module")
def capi():
    lib = os.path.join(PKG, "fa_mi355x", "lib", "libfa_mi355x.so")
    if not os.path.exists(lib):
        subprocess.run([sys.executable, os.path.join(PKG, "build.py")], check=True)
    from fa_mi355x import capi as c
    return c


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(fa_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol(capi):
    names = header_functions()
    assert len(names) >= 8, names
    lib = ctypes.CDLL(capi.CORE_LIB)
    for n in names:
        assert hasattr(lib, n), f"libfa_mi355x.so does not export {n}"
    assert sorted(capi.EXPORTED) == names
    assert capi.lib().fa_abi_version() == capi.ABI_VERSION == 4


@pytest.mark.parametrize("struct", ["fa_fwd_params", "fa_bwd_params"])
def test_params_layout_matches_header(capi, tmp_path, struct):
    """Compile a probe against the header and compare sizeof/offsetof of every
    field with the ctypes mirror."""
    mirror = {"fa_fwd_params": capi.FwdParams, "fa_bwd_params": capi.BwdParams}[struct]
    fields = [n for n, _ in mirror._fields_]
    src = tmp_path / "probe.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "fa_mi355x.h"', "int main(void) {",
             f'  printf("size %zu\\n", sizeof({struct}));']
    for n in fields:
        lines.append(f'  printf("{n} %zu\\n", offsetof({struct}, {n}));')
    lines.append("  return 0; }")
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)], check=True)
    out = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True, check=True)
               .stdout.splitlines())
    assert int(out["size"]) == ctypes.sizeof(mirror)
    for n in fields:
        assert int(out[n]) == getattr(mirror, n).offset, n


def _valid_bwd(capi, **kw):
    """A dense backward description with fake (aligned, never dereferenced) pointers."""
    base = dict(dtype=capi.FA_DTYPE_FP16, batch=2, seqlen_q=64, seqlen_k=96, nheads=8, nheads_k=2, headdim=128,
                softmax_scale=0.088, is_causal=1, softmax_lse=0x90000, softmax_d=0xa0000)
    for i, n in enumerate(["q", "k", "v", "out", "dout", "dq", "dk", "dv"]):
        heads = 2 if n in ("k", "v", "dk", "dv") else 8
        seq = 96 if n in ("k", "v", "dk", "dv") else 64
        base.update({n: 0x10000 * (i + 1), f"{n}_batch_stride": seq * heads * 128, f"{n}_row_stride": heads * 128,
                     f"{n}_head_stride": 128})
    base.update(kw)
    return capi.new_bwd_params(**base)


def test_validate_bwd(capi):
    assert capi.validate_bwd(_valid_bwd(capi), capi.FA_KIND_DENSE) == capi.FA_OK
    for d in (64, 136, 192, 256):
        assert capi.validate_bwd(_valid_bwd(capi, headdim=d), capi.FA_KIND_DENSE) == capi.FA_OK, d
    bad = [
        (dict(dropout_p=0.1), capi.FA_KIND_DENSE, capi.FA_EUNSUPPORTED, "dropout"),
        (dict(headdim=264), capi.FA_KIND_DENSE, capi.FA_EINVAL, "at most 256"),
        (dict(nheads_k=3), capi.FA_KIND_DENSE, capi.FA_EINVAL, "must divide"),
        (dict(softcap=-1.0), capi.FA_KIND_DENSE, capi.FA_EINVAL, "softcap"),
        (dict(dq=0x10008), capi.FA_KIND_DENSE, capi.FA_EINVAL, "16-byte aligned"),
        (dict(softmax_d=None), capi.FA_KIND_DENSE, capi.FA_EINVAL, "softmax_d"),
        (dict(attention_chunk=-1), capi.FA_KIND_DENSE, capi.FA_EINVAL, "attention_chunk"),
        (dict(), capi.FA_KIND_VARLEN, capi.FA_EINVAL, "cu_seqlens_q and cu_seqlens_k are required"),
        (dict(), capi.FA_KIND_KVCACHE, capi.FA_EINVAL, "dense or varlen"),
        (dict(dtype=capi.FA_DTYPE_FP8_E4M3), capi.FA_KIND_DENSE, capi.FA_EINVAL, "only support fp16 and bf16"),
    ]
    for kw, kind, code, msg in bad:
        assert capi.validate_bwd(_valid_bwd(capi, **kw), kind) == code, kw
        assert msg in capi.last_error(), (kw, capi.last_error())


def _valid(capi, **kw):
    """A kvcache decode description with fake (aligned, never dereferenced) pointers."""
    base = dict(dtype=capi.FA_DTYPE_BF16, batch=2, seqlen_q=1, nheads=8, nheads_k=2, headdim=128, headdim_v=128,
                seqlen_k=256, batch_cache=2, q=0x10000, q_batch_stride=1024, q_row_stride=1024, q_head_stride=128,
                k=0x20000, k_batch_stride=256 * 256, k_row_stride=256, k_head_stride=128,
                v=0x30000, v_batch_stride=256 * 256, v_row_stride=256, v_head_stride=128,
                out=0x40000, out_batch_stride=1024, out_row_stride=1024, out_head_stride=128,
                softmax_lse=ctypes.cast(0x50000, ctypes.c_void_p), cache_seqlens=0x60000, softmax_scale=0.088,
                is_causal=1)
    base.update(kw)
    return capi.new_params(**base)


def test_validate_accepts_a_valid_call(capi):
    assert capi.validate(_valid(capi), capi.FA_KIND_KVCACHE) == capi.FA_OK
    for d in (8, 64, 96, 128, 136, 192, 256):
        assert capi.validate(_valid(capi, headdim=d, headdim_v=d), capi.FA_KIND_DENSE) == capi.FA_OK, d
    assert capi.validate(_valid(capi, k_new=0x70000, v_new=0x80000, seqlen_new=1, knew_batch_stride=256,
                                knew_row_stride=256, knew_head_stride=128, vnew_batch_stride=256,
                                vnew_row_stride=256, vnew_head_stride=128), capi.FA_KIND_KVCACHE) == capi.FA_OK
    # v3 kvcache extensions: ragged q and new tokens, leftpad, rotary positions, chunked attention
    assert capi.validate(_valid(capi, k_new=0x70000, v_new=0x80000, cu_seqlens_k_new=0xE0000, total_k_new=5,
                                knew_row_stride=256, knew_head_stride=128, vnew_row_stride=256,
                                vnew_head_stride=128, cu_seqlens_q=0xF0000, total_q=7, cache_leftpad=0xD0000,
                                attention_chunk=64), capi.FA_KIND_KVCACHE) == capi.FA_OK
    assert capi.validate(_valid(capi, attention_chunk=128), capi.FA_KIND_DENSE) == capi.FA_OK
    # FP8 (e4m3) inputs with per (batch, kv head) descales; headdim a multiple of 16
    for d in (64, 96, 128, 192, 256):
        assert capi.validate(_valid(capi, dtype=capi.FA_DTYPE_FP8_E4M3, headdim=d, headdim_v=d,
                                    q_descale=0x11000, q_descale_batch_stride=2, q_descale_head_stride=1,
                                    k_descale=0x12000, v_descale=0x13000), capi.FA_KIND_DENSE) == capi.FA_OK, d


QV = dict(qv=0x15000, qv_batch_stride=1024, qv_row_stride=1024, qv_head_stride=128)


def test_validate_qv_where_the_decode_kernel_runs(capi):
    # rows per kv head = seqlen_q * nheads / nheads_k with packed GQA, seqlen_q without
    assert capi.validate(_valid(capi, seqlen_q=4, **QV), capi.FA_KIND_KVCACHE) == capi.FA_OK, capi.last_error()
    assert capi.validate(_valid(capi, seqlen_q=2, **QV), capi.FA_KIND_DENSE) == capi.FA_OK, capi.last_error()
    assert capi.validate(_valid(capi, seqlen_q=16, no_pack_gqa=1, **QV), capi.FA_KIND_KVCACHE) == capi.FA_OK
    assert capi.validate(_valid(capi, seqlen_q=16, **QV), capi.FA_KIND_KVCACHE) == capi.FA_EUNSUPPORTED


BAD = [
    # (field overrides, kind, expected status, message fragment)
    (dict(abi_version=7), 0, "EINVAL", "abi_version"),
    (dict(dtype=2), 0, "EINVAL", "only support fp16 and bf16"),
    (dict(nheads=6, nheads_k=4), 0, "EINVAL", "must divide number of heads in query"),
    (dict(headdim=264, headdim_v=264), 0, "EINVAL", "at most 256"),
    (dict(headdim=60, headdim_v=60), 0, "EINVAL", "multiple of 8"),
    (dict(dropout_p=0.1), 1, "EUNSUPPORTED", "dropout"),
    (dict(q=0x10008), 0, "EINVAL", "16-byte aligned"),
    (dict(k_row_stride=250), 0, "EINVAL", "k strides"),
    (dict(k_new=0x70000, seqlen_new=1), 0, "EINVAL", "value must also be passed in"),
    (dict(rotary_cos=0x90000, rotary_sin=0xA0000, rotary_dim=64, seqlen_ro=16), 0, "EINVAL",
     "new key / value to be appended"),
    (dict(batch=0), 0, "EINVAL", "batch size"),
    (dict(softcap=-1.0), 0, "EINVAL", "softcap"),
    (dict(batch_cache=1), 0, "EINVAL", "smaller than q batch"),
    (dict(block_table=0xB0000, page_block_size=0, max_blocks_per_seq=1, block_table_rows=2), 0, "EINVAL",
     "page_block_size"),
    (dict(alibi_slopes=ctypes.cast(0xC0000, ctypes.c_void_p), alibi_batch_stride=3), 0, "EINVAL", "alibi_slopes"),
    (dict(), 2, "EINVAL", "cu_seqlens_q is required"),
    (dict(block_table=0xB0000, page_block_size=16, max_blocks_per_seq=1), 1, "EINVAL", "dense forward"),
    (dict(attention_chunk=-4), 1, "EINVAL", "attention_chunk"),
    (dict(cache_leftpad=0xD0000, block_table=0xB0000, page_block_size=16, max_blocks_per_seq=1,
          block_table_rows=2), 0, "EINVAL", "cache_leftpad is not supported with a paged"),
    (dict(cu_seqlens_k_new=0xE0000, total_k_new=3), 0, "EINVAL", "without new keys"),
    (dict(cache_leftpad=0xD0000), 1, "EINVAL", "only valid for the kvcache forward"),
    (dict(cu_seqlens_q=0xF0000, total_q=-1), 0, "EINVAL", "total_q must be >= 0"),
    (dict(dtype=3, headdim=72, headdim_v=72), 1, "EINVAL", "multiple of 16"),
    (dict(dtype=3, k_row_stride=264), 0, "EINVAL", "FP8 q, k and v strides"),
    (dict(dtype=3, k_new=0x70000, v_new=0x80000, seqlen_new=1, knew_batch_stride=256, knew_row_stride=256,
          knew_head_stride=128, vnew_batch_stride=256, vnew_row_stride=256, vnew_head_stride=128,
          rotary_cos=0x90000, rotary_sin=0xA0000, rotary_dim=64, seqlen_ro=16), 0, "EINVAL",
     "rotary is not supported with FP8"),
    (dict(dtype=4), 1, "EINVAL", "only support fp16 and bf16"),
    (dict(dtype=3, **QV), 0, "EINVAL", "qv is not supported with FP8"),
    (dict(QV, qv=0x15008), 0, "EINVAL", "qv must be 16-byte aligned"),
    (dict(QV, qv_row_stride=1020), 0, "EINVAL", "qv must be 16-byte aligned"),
    (dict(seqlen_q=5, **QV), 0, "EUNSUPPORTED", "qv is supported where the decode kernel runs"),
    (dict(headdim=192, headdim_v=192, **QV), 1, "EUNSUPPORTED", "qv is supported where the decode kernel runs"),
]


@pytest.mark.parametrize("over,kind,status,frag", BAD, ids=[b[3] for b in BAD])
def test_validate_rejects(capi, over, kind, status, frag):
    p = _valid(capi, **over)
    st = capi.validate(p, kind)
    assert st == getattr(capi, "FA_" + status), (st, capi.last_error())
    assert frag in capi.last_error()


def test_large_batch_accepted(capi):
    # batches above 2048 run their attention in chunks of launches; the
    # workspace is sized for one chunk
    p = _valid(capi, batch=4096, batch_cache=4096)
    assert capi.validate(p, 0) == capi.FA_OK, capi.last_error()
    st, big = capi.workspace_size(p, 0)
    assert st == capi.FA_OK, capi.last_error()
    p2 = _valid(capi, batch=2048, batch_cache=2048)
    st, one = capi.workspace_size(p2, 0)
    assert st == capi.FA_OK and big == one


def test_operators_have_meta_shapes():
    import fa_mi355x
    ops = fa_mi355x.ops
    m = "meta"
    q = torch.empty(2, 3, 8, 128, dtype=torch.bfloat16, device=m)
    kc = torch.empty(2, 64, 2, 128, dtype=torch.bfloat16, device=m)
    o, l = ops.fwd_kvcache(q, kc, kc, None, None, None, None, None, None, None, None, None, 0.1, True, -1, 0, 0.0,
                           True, 0)
    assert o.shape == q.shape and l.shape == (2, 8, 3) and l.dtype == torch.float32
    o, l = ops.fwd(q, kc, kc, None, 0.0, 0.1, True, -1, 0, 0.0)
    assert o.shape == q.shape and l.shape == (2, 8, 3)
    qv = torch.empty(10, 8, 128, dtype=torch.float16, device=m)
    kv = torch.empty(20, 2, 128, dtype=torch.float16, device=m)
    cu = torch.empty(3, dtype=torch.int32, device=m)
    o, l = ops.varlen_fwd(qv, kv, kv, cu, cu, None, None, None, 5, 10, 0.0, 0.1, True, -1, 0, 0.0)
    assert o.shape == qv.shape and l.shape == (8, 10)
    op = torch.empty(4, 2, 3, 8, 128, dtype=torch.float32, device=m)
    lp = torch.empty(4, 2, 3, 8, dtype=torch.float32, device=m)
    o, l = ops.fwd_combine(op, lp, torch.bfloat16)
    assert o.shape == (2, 3, 8, 128) and o.dtype == torch.bfloat16 and l.shape == (2, 3, 8)
    l = ops.fwd_combine_out(op, lp, torch.empty(2, 3, 8, 128, dtype=torch.float16, device=m))
    assert l.shape == (2, 3, 8) and l.dtype == torch.float32
    # FP8 (e4m3) inputs give a bf16 out in every forward op, v2 kvcache included
    q8 = torch.empty(2, 3, 8, 128, dtype=torch.float8_e4m3fn, device=m)
    k8 = torch.empty(2, 64, 2, 128, dtype=torch.float8_e4m3fn, device=m)
    o, _ = ops.fwd_kvcache(q8, k8, k8, None, None, None, None, None, None, None, None, None, 0.1, True, -1, 0, 0.0,
                           True, 0)
    assert o.dtype == torch.bfloat16
    o, _ = ops.fwd(q8, k8, k8, None, 0.0, 0.1, True, -1, 0, 0.0)
    assert o.dtype == torch.bfloat16


def test_no_cpu_fallback():
    """The public APIs run only the HIP kernels: CPU tensors raise instead of
    silently computing somewhere else."""
    import flash_attn_npu_v2
    q = torch.randn(1, 1, 4, 128, dtype=torch.bfloat16)
    kc = torch.randn(1, 16, 1, 128, dtype=torch.bfloat16)
    with pytest.raises((RuntimeError, NotImplementedError)):
        flash_attn_npu_v2.flash_attn_with_kvcache(q, kc, kc, cache_seqlens=4, causal=True)
    with pytest.raises((RuntimeError, NotImplementedError)):
        flash_attn_npu_v2.flash_attn_func(q, kc, kc, causal=True)
