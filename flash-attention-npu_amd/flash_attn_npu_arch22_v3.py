"""The reference's compiled v3 module, flash_attn_npu_arch22_v3, as a drop-in
over the MI355X implementation, with the pybind11 bindings' positional
arguments and return lists (csrc/arch22/flash_attn_npu_v3/flash_api.cpp:
816-822, called positionally by flash_attn_npu_v3/interface_arch22.py:111-146,
:294-318, :931 and :1119-1138):

  fwd                    <- mha_fwd (:60-98): dense, varlen or kvcache by its arguments
                            -> [out, softmax_lse, out_accum, softmax_lse_accum]
  bwd                    <- mha_bwd (:560-582) -> [dq, dk, dv, softmax_d]
  get_scheduler_metadata <- get_scheduler_metadata (:493-517)
  fwd_combine            <- the combine the reference's flash_attn_combine calls (:931)

fwd routes the way the reference's Python layer calls it: cu_seqlens_k means
flash_attn_varlen_func, a cache length (seqused_k), page table or new k / v
without cu_seqlens_k means flash_attn_with_kvcache, and neither means
flash_attn_func."""
import torch

import flash_attn_npu_v3 as _v3
from fa_mi355x import ops


def fwd(q, k, v, k_new, v_new, qv, out_, cu_seqlens_q, cu_seqlens_k, cu_seqlens_k_new, seqused_q, seqused_k,
        max_seqlen_q, max_seqlen_k, page_table, kv_batch_idx, leftpad_k, rotary_cos, rotary_sin, seqlens_rotary,
        q_descale, k_descale, v_descale, softmax_scale, is_causal, window_size_left, window_size_right,
        attention_chunk, softcap, is_rotary_interleaved, scheduler_metadata, num_splits, pack_gqa, sm_margin):
    window = (int(window_size_left), int(window_size_right))
    common = dict(softmax_scale=softmax_scale, causal=bool(is_causal), window_size=window,
                  attention_chunk=int(attention_chunk), softcap=float(softcap), num_splits=int(num_splits),
                  pack_gqa=pack_gqa, sm_margin=sm_margin, scheduler_metadata=scheduler_metadata, q_descale=q_descale,
                  k_descale=k_descale, v_descale=v_descale, qv=qv)
    if cu_seqlens_k is not None:
        out, lse = _v3.flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                                              seqused_q=seqused_q, seqused_k=seqused_k, return_attn_probs=True,
                                              **common)
    elif seqused_k is not None or page_table is not None or k_new is not None:
        out, lse, *_ = _v3.flash_attn_with_kvcache(q, k, v, k=k_new, v=v_new, rotary_cos=rotary_cos,
                                                   rotary_sin=rotary_sin, cache_seqlens=seqused_k,
                                                   cache_batch_idx=kv_batch_idx, cache_leftpad=leftpad_k,
                                                   page_table=page_table, cu_seqlens_q=cu_seqlens_q,
                                                   cu_seqlens_k_new=cu_seqlens_k_new, max_seqlen_q=max_seqlen_q,
                                                   rotary_seqlens=seqlens_rotary,
                                                   rotary_interleaved=bool(is_rotary_interleaved),
                                                   return_softmax_lse=True, **common)
    else:
        if seqused_q is not None:
            raise RuntimeError("seqused_q is not supported by flash_attn_npu_v3 on MI355X")
        out, lse = _v3.flash_attn_func(q, k, v, return_attn_probs=True, **common)
    if out_ is not None:
        out_.copy_(out)
        out = out_
    e = torch.empty((0,), dtype=torch.float32, device=out.device)
    return [out, lse, e, e]


def bwd(dout, q, k, v, out, softmax_lse, dq_, dk_, dv_, cu_seqlens_q, cu_seqlens_k, seqused_q, seqused_k,
        max_seqlen_q, max_seqlen_k, softmax_scale, is_causal, window_size_left, window_size_right, softcap,
        deterministic, sm_margin):
    if seqused_q is not None or seqused_k is not None:
        raise RuntimeError("seqused_q / seqused_k are not supported by the backward on MI355X")
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** (-0.5)
    if cu_seqlens_q is not None:
        dq, dk, dv, sd = ops.varlen_bwd(dout, q, k, v, out, softmax_lse, cu_seqlens_q, cu_seqlens_k, None,
                                        int(max_seqlen_q), int(max_seqlen_k), 0.0, float(softmax_scale),
                                        bool(is_causal), int(window_size_left), int(window_size_right), float(softcap),
                                        bool(deterministic))
    else:
        dq, dk, dv, sd = ops.bwd(dout, q, k, v, out, softmax_lse, None, 0.0, float(softmax_scale), bool(is_causal),
                                 int(window_size_left), int(window_size_right), float(softcap), bool(deterministic))
    outs = []
    for dst, src in ((dq_, dq), (dk_, dk), (dv_, dv)):
        if dst is not None:
            dst.copy_(src)
            src = dst
        outs.append(src)
    return outs + [sd]


def get_scheduler_metadata(batch_size, max_seqlen_q, max_seqlen_k, num_heads_q, num_heads_kv, headdim, headdim_v,
                           qkv_dtype, cache_seqlens, cu_seqlens_q, cu_seqlens_k, cu_seqlens_k_new, seqused_q,
                           cache_leftpad, page_size, max_seqlen_k_new, causal, window_size_left, window_size_right,
                           attention_chunk, has_softcap, num_splits, pack_gqa, sm_margin):
    return _v3.get_scheduler_metadata(batch_size, max_seqlen_q, max_seqlen_k, num_heads_q, num_heads_kv, headdim,
                                      cache_seqlens, qkv_dtype=qkv_dtype, headdim_v=headdim_v,
                                      cu_seqlens_q=cu_seqlens_q, cu_seqlens_k_new=cu_seqlens_k_new,
                                      cache_leftpad=cache_leftpad, page_size=page_size,
                                      max_seqlen_k_new=max_seqlen_k_new, causal=causal,
                                      window_size=(window_size_left, window_size_right),
                                      attention_chunk=attention_chunk, has_softcap=has_softcap,
                                      num_splits=num_splits, pack_gqa=pack_gqa, sm_margin=sm_margin)


def fwd_combine(out_partial, lse_partial, out=None, out_dtype=None):
    return _v3.flash_attn_combine(out_partial, lse_partial, out=out, out_dtype=out_dtype)
