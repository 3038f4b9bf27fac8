"""v3 FlashAttention API (forward) over the MI355X operators.

Names, keywords, defaults and return arity follow the reference
(flash_attn_npu_v3/interface_arch22.py): flash_attn_func :797-877,
flash_attn_varlen_func :880-927, flash_attn_combine :930-931,
flash_attn_with_kvcache :934-1095, get_scheduler_metadata :1098-1138.
The reference routes all three through one custom op (:63-154); here each
maps onto the matching fa_mi355x operator. flash_attn_func and
flash_attn_varlen_func have a backward (the reference's :536-698 autograd
Functions), run by the MI355X backward kernels.

FP8: q, k, v (and the cache, k / v of flash_attn_with_kvcache) may be
torch.float8_e4m3fn with q_descale / k_descale / v_descale of shape
(batch_size, nheads_k) fp32; scores are scaled by q_descale * k_descale and
the output by v_descale, and out is bf16 (forward only, no rotary). The
reference rejects the descales (csrc/arch22/flash_attn_npu_v3/
flash_api.cpp:154-156).
"""
from typing import Optional, Union

import torch

from fa_mi355x import ops


def maybe_contiguous(x):
    return x.contiguous() if x is not None and x.stride(-1) != 1 else x


def _reject(**kw):
    for name, val in kw.items():
        if val is not None and val is not False and not (isinstance(val, (int, float)) and val == 0):
            raise RuntimeError(f"{name} is not supported by flash_attn_npu_v3 on MI355X")


def _empty_accum(out):
    e = torch.empty((0,), dtype=torch.float32, device=out.device)
    return e, e


def _check_metadata(scheduler_metadata, device):
    # The split-KV plan is made on the device from cache_seqlens inside the
    # attention kernel, so a precomputed plan only has to describe the same
    # problem; results are identical with or without it.
    if scheduler_metadata is not None and scheduler_metadata.device != device:
        raise RuntimeError("scheduler_metadata must be on the same device as q")


def _cu_from_lengths(lengths):
    z = torch.zeros((1,), dtype=torch.int32, device=lengths.device)
    return torch.cat([z, torch.cumsum(lengths, 0, dtype=torch.int32)])


class FlashAttnFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, softmax_scale, causal, qv=None, q_descale=None, k_descale=None, v_descale=None,
                window_size=(-1, -1), attention_chunk=0, softcap=0.0, num_splits=1, pack_gqa=None,
                deterministic=False, sm_margin=0, return_softmax=False, scheduler_metadata=None):
        _reject(qv=qv)
        if softmax_scale is None:
            softmax_scale = q.shape[-1] ** (-0.5)
        _check_metadata(scheduler_metadata, q.device)
        q, k, v = [maybe_contiguous(x) for x in (q, k, v)]
        out, softmax_lse = ops.fwd(q, k, v, None, 0.0, float(softmax_scale), bool(causal), int(window_size[0]),
                                   int(window_size[1]), float(softcap), int(attention_chunk), q_descale, k_descale,
                                   v_descale)
        if any(x.requires_grad for x in (q, k, v)):
            ctx.save_for_backward(q, k, v, out, softmax_lse)
            ctx.softmax_scale = softmax_scale
            ctx.causal = causal
            ctx.window_size = window_size
            ctx.softcap = softcap
            ctx.deterministic = deterministic
            ctx.attention_chunk = attention_chunk
        return (out, softmax_lse) if return_softmax else out

    @staticmethod
    def backward(ctx, dout, *args):
        q, k, v, out, softmax_lse = ctx.saved_tensors
        dq, dk, dv, _ = ops.bwd(maybe_contiguous(dout), q, k, v, out, softmax_lse, None, 0.0,
                                float(ctx.softmax_scale), bool(ctx.causal), int(ctx.window_size[0]),
                                int(ctx.window_size[1]), float(ctx.softcap), bool(ctx.deterministic),
                                int(ctx.attention_chunk))
        return (dq, dk, dv) + (None,) * 15


class FlashAttnVarlenFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_q, seqused_k, max_seqlen_q, max_seqlen_k,
                softmax_scale, causal, qv=None, q_descale=None, k_descale=None, v_descale=None, window_size=(-1, -1),
                attention_chunk=0, softcap=0.0, num_splits=1, pack_gqa=None, deterministic=False, sm_margin=0,
                return_softmax=False, scheduler_metadata=None):
        _reject(seqused_q=seqused_q, qv=qv)
        if softmax_scale is None:
            softmax_scale = q.shape[-1] ** (-0.5)
        _check_metadata(scheduler_metadata, q.device)
        q, k, v = [maybe_contiguous(x) for x in (q, k, v)]
        out, softmax_lse = ops.varlen_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, None, None,
                                          int(max_seqlen_q), int(max_seqlen_k), 0.0, float(softmax_scale),
                                          bool(causal), int(window_size[0]), int(window_size[1]), float(softcap),
                                          int(attention_chunk), q_descale, k_descale, v_descale)
        if any(x.requires_grad for x in (q, k, v)):
            ctx.save_for_backward(q, k, v, out, softmax_lse, cu_seqlens_q, cu_seqlens_k)
            ctx.has_seqused_k = seqused_k is not None
            ctx.max_seqlen_q = max_seqlen_q
            ctx.max_seqlen_k = max_seqlen_k
            ctx.softmax_scale = softmax_scale
            ctx.causal = causal
            ctx.window_size = window_size
            ctx.softcap = softcap
            ctx.deterministic = deterministic
            ctx.attention_chunk = attention_chunk
        return (out, softmax_lse) if return_softmax else out

    @staticmethod
    def backward(ctx, dout, *args):
        if ctx.has_seqused_k:
            raise RuntimeError("flash_attn_varlen_func has no backward with seqused_k")
        q, k, v, out, softmax_lse, cu_seqlens_q, cu_seqlens_k = ctx.saved_tensors
        dq, dk, dv, _ = ops.varlen_bwd(maybe_contiguous(dout), q, k, v, out, softmax_lse, cu_seqlens_q, cu_seqlens_k,
                                       None, int(ctx.max_seqlen_q), int(ctx.max_seqlen_k), 0.0,
                                       float(ctx.softmax_scale), bool(ctx.causal), int(ctx.window_size[0]),
                                       int(ctx.window_size[1]), float(ctx.softcap), bool(ctx.deterministic),
                                       int(ctx.attention_chunk))
        return (dq, dk, dv) + (None,) * 21


def flash_attn_func(q, k, v, softmax_scale=None, causal=False, qv=None, q_descale=None, k_descale=None,
                    v_descale=None, window_size=(-1, -1), attention_chunk=0, softcap=0.0, num_splits=1, pack_gqa=None,
                    deterministic=False, sm_margin=0, return_attn_probs=False, scheduler_metadata=None):
    """q: (batch_size, seqlen, nheads, headdim); k, v: (batch_size, seqlen, nheads_k, headdim).
    Returns out, or (out, softmax_lse (batch, nheads, seqlen)) when return_attn_probs."""
    return FlashAttnFunc.apply(q, k, v, softmax_scale, causal, qv, q_descale, k_descale, v_descale, window_size,
                               attention_chunk, softcap, num_splits, pack_gqa, deterministic, sm_margin,
                               return_attn_probs, scheduler_metadata)


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, seqused_q=None,
                           seqused_k=None, softmax_scale=None, causal=False, qv=None, q_descale=None, k_descale=None,
                           v_descale=None, window_size=(-1, -1), attention_chunk=0, softcap=0.0, num_splits=1,
                           pack_gqa=None, deterministic=False, sm_margin=0, return_attn_probs=False,
                           scheduler_metadata=None):
    """q: (total_q, nheads, headdim); k, v: (total_k, nheads_k, headdim).
    softmax_lse is (nheads, total_q)."""
    return FlashAttnVarlenFunc.apply(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_q, seqused_k, max_seqlen_q,
                                     max_seqlen_k, softmax_scale, causal, qv, q_descale, k_descale, v_descale,
                                     window_size, attention_chunk, softcap, num_splits, pack_gqa, deterministic,
                                     sm_margin, return_attn_probs, scheduler_metadata)


def flash_attn_combine(out_partial, lse_partial, out=None, out_dtype=None):
    """Merge split-KV partials: out_partial (num_splits, ..., headdim_v) fp32 and
    lse_partial (num_splits, ...) fp32 -> (out, lse) with
    lse = log sum_s exp(lse_s) and out = sum_s exp(lse_s - lse) out_s."""
    return ops.fwd_combine(out_partial, lse_partial, out, out_dtype)


def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, qv=None, rotary_cos=None, rotary_sin=None,
                            cache_seqlens: Optional[Union[int, torch.Tensor]] = None,
                            cache_batch_idx: Optional[torch.Tensor] = None,
                            cache_leftpad: Optional[torch.Tensor] = None, page_table: Optional[torch.Tensor] = None,
                            cu_seqlens_q: Optional[torch.Tensor] = None,
                            cu_seqlens_k_new: Optional[torch.Tensor] = None, max_seqlen_q: Optional[int] = None,
                            rotary_seqlens: Optional[torch.Tensor] = None, q_descale: Optional[torch.Tensor] = None,
                            k_descale: Optional[torch.Tensor] = None, v_descale: Optional[torch.Tensor] = None,
                            softmax_scale=None, causal=False, window_size=(-1, -1), attention_chunk=0, softcap=0.0,
                            rotary_interleaved=True, scheduler_metadata=None, num_splits=0, pack_gqa=None,
                            sm_margin=0, return_softmax_lse=False):
    """Attention against a KV cache (optionally appending k/v in place first).

    q: (batch_size, seqlen, nheads, headdim) or, with cu_seqlens_q,
    (total_q, nheads, headdim). k_cache/v_cache: (batch_size_cache,
    seqlen_cache, nheads_k, headdim), (num_blocks, page_block_size, nheads_k,
    headdim) with page_table, or with cu_seqlens_q and no page_table a packed
    (total_k, nheads_k, headdim) cache indexed by the prefix sums of
    cache_seqlens. k / v (appended in place at cache_seqlens) are (batch_size,
    seqlen_new, nheads_k, headdim), or (total_k_new, nheads_k, headdim) split
    by cu_seqlens_k_new. cache_leftpad[b] is the first valid cache row of
    sequence b (contiguous caches). Rotary positions start at rotary_seqlens[b]
    (default cache_seqlens[b]). attention_chunk > 0 restricts each query to
    the keys of its own chunk of that size. With float8_e4m3fn q / caches / k / v,
    q_descale, k_descale and v_descale ((batch_size, nheads_k) fp32) scale the
    scores and the output, and out is bf16. Returns out, or (out, softmax_lse,
    out_accum, lse_accum) when return_softmax_lse (the accumulators are empty
    tensors)."""
    assert k_cache.stride(-1) == 1, "k_cache must have contiguous last dimension"
    assert v_cache.stride(-1) == 1, "v_cache must have contiguous last dimension"
    _reject(qv=qv)
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** (-0.5)
    batch = q.shape[0] if cu_seqlens_q is None else cu_seqlens_q.numel() - 1
    if cache_seqlens is not None and isinstance(cache_seqlens, int):
        cache_seqlens = torch.full((batch,), cache_seqlens, dtype=torch.int32, device=k_cache.device)
    cache_seqlens = maybe_contiguous(cache_seqlens)
    _check_metadata(scheduler_metadata, q.device)
    q, k, v = [maybe_contiguous(x) for x in (q, k, v)]
    if cu_seqlens_q is not None and max_seqlen_q is None:
        raise RuntimeError("max_seqlen_q is required with cu_seqlens_q")
    if cu_seqlens_q is not None and page_table is None and k_cache.dim() == 3:
        # varlen (TND) queries against a packed (total_k, nheads_k, headdim)
        # cache indexed by the prefix sums of cache_seqlens
        # (csrc/arch22/flash_attn_npu_v3/flash_api.cpp:431-441 in the reference)
        _reject(k=k, v=v, rotary_cos=rotary_cos, cache_batch_idx=cache_batch_idx, cache_leftpad=cache_leftpad,
                cu_seqlens_k_new=cu_seqlens_k_new)
        if cache_seqlens is None:
            raise RuntimeError("cache_seqlens is required with cu_seqlens_q")
        cu_k = _cu_from_lengths(cache_seqlens)
        out, softmax_lse = ops.varlen_fwd(q, k_cache, v_cache, cu_seqlens_q, cu_k, cache_seqlens, None, None,
                                          int(max_seqlen_q), int(k_cache.shape[0]), 0.0, float(softmax_scale),
                                          bool(causal), int(window_size[0]), int(window_size[1]), float(softcap),
                                          int(attention_chunk), q_descale, k_descale, v_descale)
    else:
        # (batch, seqlen) or ragged (total_q) queries against a (batch_cache,
        # seqlen_cache) or paged cache, with the in-place append of k / v
        # (ragged with cu_seqlens_k_new), rotary at rotary_seqlens (default
        # cache_seqlens), cache_leftpad and attention_chunk
        out, softmax_lse = ops.fwd_kvcache_v3(q, k_cache, v_cache, k, v, cache_seqlens, rotary_cos, rotary_sin,
                                              maybe_contiguous(cache_batch_idx), maybe_contiguous(cache_leftpad),
                                              maybe_contiguous(page_table), None, cu_seqlens_q, cu_seqlens_k_new,
                                              int(max_seqlen_q or 0), maybe_contiguous(rotary_seqlens),
                                              float(softmax_scale), bool(causal), int(window_size[0]),
                                              int(window_size[1]), int(attention_chunk), float(softcap),
                                              bool(rotary_interleaved), int(num_splits), q_descale, k_descale,
                                              v_descale)
    if return_softmax_lse:
        oa, la = _empty_accum(out)
        return out, softmax_lse, oa, la
    return out


def get_scheduler_metadata(batch_size, max_seqlen_q, max_seqlen_k, num_heads_q, num_heads_kv, headdim,
                           cache_seqlens: torch.Tensor, qkv_dtype=torch.bfloat16, headdim_v=None,
                           cu_seqlens_q: Optional[torch.Tensor] = None,
                           cu_seqlens_k_new: Optional[torch.Tensor] = None,
                           cache_leftpad: Optional[torch.Tensor] = None, page_size: Optional[int] = None,
                           max_seqlen_k_new=0, causal=False, window_size=(-1, -1), attention_chunk=0,
                           has_softcap=False, num_splits=0, pack_gqa=None, sm_margin=0):
    """Describes the problem for a later flash_attn_with_kvcache call.

    On MI355X the split-KV plan is computed by the attention kernel itself from
    cache_seqlens (no host synchronisation), so the metadata is a small int32
    descriptor of the problem shape on the device of cache_seqlens; passing it
    back does not change results (the reference contract:
    tests/test_flash_attn_npu_v3_metadata.py)."""
    if headdim_v is None:
        headdim_v = headdim
    desc = [1, batch_size, max_seqlen_q, max_seqlen_k, num_heads_q, num_heads_kv, headdim, headdim_v,
            int(bool(causal)), int(window_size[0]), int(window_size[1]), int(num_splits), page_size or 0]
    return torch.tensor(desc, dtype=torch.int32, device=cache_seqlens.device)
