"""v2 FlashAttention API (forward) over the MI355X operators.

Function names, keywords, defaults and return arity follow the reference
(flash_attn_npu_v2/interface_arch22.py): flash_attn_func :1102-1176,
flash_attn_varlen_func :1337-1428, flash_attn_with_kvcache :1431-1573, the
packed variants :965-1336 and the autograd Functions :407-962.

The backward of flash_attn_func / flash_attn_varlen_func (and the packed
variants built on them) runs the MI355X backward kernels
(interface_arch22.py:204-404,827-857 in the reference); dropout and a paged
k/v (block_table) have no backward.
"""
from typing import Optional, Union

import torch

from fa_mi355x import ops


def maybe_contiguous(x):
    return x.contiguous() if x is not None and x.stride(-1) != 1 else x


def _pad8(x, head_size_og):
    return torch.nn.functional.pad(x, [0, 8 - head_size_og % 8]) if head_size_og % 8 != 0 else x


def _flash_attn_forward(q, k, v, dropout_p, softmax_scale, causal, window_size_left=-1, window_size_right=-1,
                        softcap=0.0, alibi_slopes=None, return_softmax=False):
    """Reference interface_arch22.py:47-77: returns (out, softmax_lse, S_dmask, rng_state)."""
    q, k, v = [maybe_contiguous(x) for x in (q, k, v)]
    out, lse = ops.fwd(q, k, v, alibi_slopes, float(dropout_p), float(softmax_scale), bool(causal),
                       int(window_size_left), int(window_size_right), float(softcap))
    s_dmask = torch.empty((0,), dtype=q.dtype, device=q.device)
    rng_state = torch.zeros((2,), dtype=torch.int64, device=q.device)
    return out, lse, s_dmask, rng_state


def _flash_attn_varlen_forward(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, dropout_p,
                               softmax_scale, causal, window_size_left=-1, window_size_right=-1, softcap=0.0,
                               alibi_slopes=None, return_softmax=False, block_table=None, leftpad_k=None,
                               seqused_k=None, zero_tensors=False):
    """Reference interface_arch22.py:113-161."""
    if leftpad_k is not None:
        raise RuntimeError("leftpad_k is not supported")
    q, k, v = [maybe_contiguous(x) for x in (q, k, v)]
    out, lse = ops.varlen_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, block_table, alibi_slopes,
                              int(max_seqlen_q),
                              int(max_seqlen_k), float(dropout_p), float(softmax_scale), bool(causal),
                              int(window_size_left), int(window_size_right), float(softcap))
    s_dmask = torch.empty((0,), dtype=q.dtype, device=q.device)
    rng_state = torch.zeros((2,), dtype=torch.int64, device=q.device)
    return out, lse, s_dmask, rng_state


def _flash_attn_backward(dout, q, k, v, out, softmax_lse, dq, dk, dv, dropout_p, softmax_scale, causal,
                         window_size_left, window_size_right, softcap, alibi_slopes, deterministic, rng_state=None):
    """Reference interface_arch22.py:204-253: fills dq, dk, dv (when given) and
    returns softmax_d = rowsum(dout * out), (batch, nheads, seqlen_q) fp32."""
    dout, q, k, v, out = [maybe_contiguous(x) for x in (dout, q, k, v, out)]
    gq, gk, gv, softmax_d = ops.bwd(dout, q, k, v, out, softmax_lse.contiguous(), alibi_slopes, float(dropout_p),
                                    float(softmax_scale), bool(causal), int(window_size_left),
                                    int(window_size_right), float(softcap), bool(deterministic))
    for dst, src in ((dq, gq), (dk, gk), (dv, gv)):
        if dst is not None:
            dst.copy_(src)
    return softmax_d if dq is not None else (gq, gk, gv, softmax_d)


def _flash_attn_varlen_backward(dout, q, k, v, out, softmax_lse, dq, dk, dv, cu_seqlens_q, cu_seqlens_k,
                                max_seqlen_q, max_seqlen_k, dropout_p, softmax_scale, causal, window_size_left,
                                window_size_right, softcap, alibi_slopes, deterministic, rng_state=None,
                                zero_tensors=False):
    """Reference interface_arch22.py:296-357."""
    dout, q, k, v, out = [maybe_contiguous(x) for x in (dout, q, k, v, out)]
    gq, gk, gv, softmax_d = ops.varlen_bwd(dout, q, k, v, out, softmax_lse.contiguous(), cu_seqlens_q,
                                           cu_seqlens_k, alibi_slopes, int(max_seqlen_q), int(max_seqlen_k),
                                           float(dropout_p), float(softmax_scale), bool(causal),
                                           int(window_size_left), int(window_size_right), float(softcap),
                                           bool(deterministic))
    for dst, src in ((dq, gq), (dk, gk), (dv, gv)):
        if dst is not None:
            dst.copy_(src)
    return softmax_d if dq is not None else (gq, gk, gv, softmax_d)


class FlashAttnFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, dropout_p, softmax_scale, causal, window_size, softcap, alibi_slopes, deterministic,
                return_softmax, is_grad_enabled):
        is_grad = is_grad_enabled and any(x.requires_grad for x in (q, k, v))
        if softmax_scale is None:
            softmax_scale = q.shape[-1] ** (-0.5)
        head_size_og = q.size(3)
        q, k, v = (_pad8(x, head_size_og) for x in (q, k, v))
        out_padded, softmax_lse, s_dmask, rng_state = _flash_attn_forward(
            q, k, v, dropout_p, softmax_scale, causal=causal, window_size_left=window_size[0],
            window_size_right=window_size[1], softcap=softcap, alibi_slopes=alibi_slopes,
            return_softmax=return_softmax and dropout_p > 0)
        if is_grad:
            ctx.save_for_backward(q, k, v, out_padded, softmax_lse, rng_state)
            ctx.dropout_p = dropout_p
            ctx.softmax_scale = softmax_scale
            ctx.causal = causal
            ctx.window_size = window_size
            ctx.softcap = softcap
            ctx.alibi_slopes = alibi_slopes
            ctx.deterministic = deterministic
        out = out_padded[..., :head_size_og]
        return out if not return_softmax else (out, softmax_lse, s_dmask)

    @staticmethod
    def backward(ctx, dout, *args):
        q, k, v, out, softmax_lse, rng_state = ctx.saved_tensors
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        head_size_og = dout.size(3)
        dout_padded = _pad8(dout, head_size_og)
        _flash_attn_backward(dout_padded, q, k, v, out, softmax_lse, dq, dk, dv, ctx.dropout_p, ctx.softmax_scale,
                             ctx.causal, ctx.window_size[0], ctx.window_size[1], ctx.softcap, ctx.alibi_slopes,
                             ctx.deterministic, rng_state=rng_state)
        dq, dk, dv = dq[..., :head_size_og], dk[..., :head_size_og], dv[..., :head_size_og]
        return dq, dk, dv, None, None, None, None, None, None, None, None, None


class FlashAttnVarlenFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, dropout_p, softmax_scale,
                causal, window_size, softcap, alibi_slopes, deterministic, return_softmax, block_table,
                is_grad_enabled):
        is_grad = is_grad_enabled and any(x.requires_grad for x in (q, k, v))
        if softmax_scale is None:
            softmax_scale = q.shape[-1] ** (-0.5)
        head_size_og = q.size(-1)
        q, k, v = (_pad8(x, head_size_og) for x in (q, k, v))
        out_padded, softmax_lse, s_dmask, rng_state = _flash_attn_varlen_forward(
            q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, dropout_p, softmax_scale,
            causal=causal, window_size_left=window_size[0], window_size_right=window_size[1], softcap=softcap,
            alibi_slopes=alibi_slopes, return_softmax=return_softmax and dropout_p > 0, block_table=block_table)
        if is_grad:
            if block_table is not None:
                raise RuntimeError("flash_attn_varlen_func has no backward with a paged k/v (block_table)")
            ctx.save_for_backward(q, k, v, out_padded, softmax_lse, cu_seqlens_q, cu_seqlens_k, rng_state)
            ctx.dropout_p = dropout_p
            ctx.max_seqlen_q = max_seqlen_q
            ctx.max_seqlen_k = max_seqlen_k
            ctx.softmax_scale = softmax_scale
            ctx.causal = causal
            ctx.window_size = window_size
            ctx.softcap = softcap
            ctx.alibi_slopes = alibi_slopes
            ctx.deterministic = deterministic
        out = out_padded[..., :head_size_og]
        return out if not return_softmax else (out, softmax_lse, s_dmask)

    @staticmethod
    def backward(ctx, dout, *args):
        q, k, v, out, softmax_lse, cu_seqlens_q, cu_seqlens_k, rng_state = ctx.saved_tensors
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        head_size_og = dout.size(2)
        dout_padded = _pad8(dout, head_size_og)
        _flash_attn_varlen_backward(dout_padded, q, k, v, out, softmax_lse, dq, dk, dv, cu_seqlens_q, cu_seqlens_k,
                                    ctx.max_seqlen_q, ctx.max_seqlen_k, ctx.dropout_p, ctx.softmax_scale, ctx.causal,
                                    ctx.window_size[0], ctx.window_size[1], ctx.softcap, ctx.alibi_slopes,
                                    ctx.deterministic, rng_state=rng_state)
        dq, dk, dv = dq[..., :head_size_og], dk[..., :head_size_og], dv[..., :head_size_og]
        return dq, dk, dv, None, None, None, None, None, None, None, None, None, None, None, None, None, None


def flash_attn_qkvpacked_func(qkv, dropout_p=0.0, softmax_scale=None, causal=False, window_size=(-1, -1),
                              softcap=0.0, alibi_slopes=None, deterministic=False, return_attn_probs=False):
    """qkv: (batch_size, seqlen, 3, nheads, headdim)."""
    q, k, v = qkv.unbind(dim=2)
    return FlashAttnFunc.apply(q, k, v, dropout_p, softmax_scale, causal, window_size, softcap, alibi_slopes,
                               deterministic, return_attn_probs, torch.is_grad_enabled())


def flash_attn_kvpacked_func(q, kv, dropout_p=0.0, softmax_scale=None, causal=False, window_size=(-1, -1),
                             softcap=0.0, alibi_slopes=None, deterministic=False, return_attn_probs=False):
    """kv: (batch_size, seqlen_k, 2, nheads_k, headdim)."""
    k, v = kv.unbind(dim=2)
    return FlashAttnFunc.apply(q, k, v, dropout_p, softmax_scale, causal, window_size, softcap, alibi_slopes,
                               deterministic, return_attn_probs, torch.is_grad_enabled())


def flash_attn_func(q, k, v, dropout_p=0.0, softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
                    alibi_slopes=None, deterministic=False, return_attn_probs=False):
    """q: (batch_size, seqlen, nheads, headdim); k, v: (batch_size, seqlen, nheads_k, headdim).

    Causal masks are aligned to the bottom-right corner; rows with no visible
    key give out = 0 and lse = +inf. Returns out, or (out, softmax_lse,
    S_dmask) when return_attn_probs (S_dmask is empty: no dropout)."""
    return FlashAttnFunc.apply(q, k, v, dropout_p, softmax_scale, causal, window_size, softcap, alibi_slopes,
                               deterministic, return_attn_probs, torch.is_grad_enabled())


def flash_attn_varlen_qkvpacked_func(qkv, cu_seqlens, max_seqlen, dropout_p=0.0, softmax_scale=None, causal=False,
                                     window_size=(-1, -1), softcap=0.0, alibi_slopes=None, deterministic=False,
                                     return_attn_probs=False):
    """qkv: (total, 3, nheads, headdim)."""
    q, k, v = qkv.unbind(dim=1)
    return FlashAttnVarlenFunc.apply(q, k, v, cu_seqlens, cu_seqlens, max_seqlen, max_seqlen, dropout_p,
                                     softmax_scale, causal, window_size, softcap, alibi_slopes, deterministic,
                                     return_attn_probs, None, torch.is_grad_enabled())


def flash_attn_varlen_kvpacked_func(q, kv, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, dropout_p=0.0,
                                    softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
                                    alibi_slopes=None, deterministic=False, return_attn_probs=False):
    """kv: (total_k, 2, nheads_k, headdim)."""
    k, v = kv.unbind(dim=1)
    return FlashAttnVarlenFunc.apply(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, dropout_p,
                                     softmax_scale, causal, window_size, softcap, alibi_slopes, deterministic,
                                     return_attn_probs, None, torch.is_grad_enabled())


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, dropout_p=0.0,
                           softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                           deterministic=False, return_attn_probs=False, block_table=None):
    """q: (total_q, nheads, headdim); k, v: (total_k, nheads_k, headdim) or, with
    block_table, (num_blocks, page_block_size, nheads_k, headdim).
    softmax_lse is (nheads, total_q)."""
    return FlashAttnVarlenFunc.apply(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, dropout_p,
                                     softmax_scale, causal, window_size, softcap, alibi_slopes, deterministic,
                                     return_attn_probs, block_table, torch.is_grad_enabled())


def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, rotary_cos=None, rotary_sin=None,
                            cache_seqlens: Optional[Union[int, torch.Tensor]] = None,
                            cache_batch_idx: Optional[torch.Tensor] = None,
                            cache_leftpad: Optional[torch.Tensor] = None,
                            block_table: Optional[torch.Tensor] = None, softmax_scale=None, causal=False,
                            window_size=(-1, -1), softcap=0.0, rotary_interleaved=True, alibi_slopes=None,
                            num_splits=0, return_softmax_lse=False):
    """Attention against a KV cache, appending k/v in place first.

    If k and v are given they are written into k_cache / v_cache at positions
    cache_seqlens[b] .. cache_seqlens[b] + seqlen_new - 1 (after rotary on k)
    and attention covers cache_seqlens[b] + seqlen_new keys. With rotary,
    q is rotated at cache_seqlens[b] + i when causal or local, else at
    cache_seqlens[b]. cache_batch_idx maps query batch b to the cache row (or
    to the block_table row for a paged cache). num_splits: 0 = heuristic,
    1 = no split, n > 1 = n chunks along the keys.
    Returns out, or (out, softmax_lse (batch, nheads, seqlen)).
    """
    assert k_cache.stride(-1) == 1, "k_cache must have contiguous last dimension"
    assert v_cache.stride(-1) == 1, "v_cache must have contiguous last dimension"
    q, k, v = [maybe_contiguous(x) for x in (q, k, v)]
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** (-0.5)
    if cache_seqlens is not None and isinstance(cache_seqlens, int):
        cache_seqlens = torch.full((q.shape[0],), cache_seqlens, dtype=torch.int32, device=k_cache.device)
        cache_seqlens = maybe_contiguous(cache_seqlens)
    cache_batch_idx = maybe_contiguous(cache_batch_idx)
    block_table = maybe_contiguous(block_table)
    out, softmax_lse = ops.fwd_kvcache(q, k_cache, v_cache, k, v, cache_seqlens, rotary_cos, rotary_sin,
                                       cache_batch_idx, cache_leftpad, block_table, alibi_slopes,
                                       float(softmax_scale), bool(causal), int(window_size[0]), int(window_size[1]),
                                       float(softcap), bool(rotary_interleaved), int(num_splits))
    return (out, softmax_lse) if return_softmax_lse else out
