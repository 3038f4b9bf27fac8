"""The reference's compiled v2 module, flash_attn_npu_arch22_v2, as a drop-in
over the MI355X operators: the same five functions with the same positional
arguments and return lists as the pybind11 bindings
(csrc/arch22/flash_attn_npu_v2/flash_api.cpp:1301-1309):

  fwd         <- mha_fwd          :628-640   -> [out, softmax_lse, p, rng_state]
  varlen_fwd  <- mha_varlen_fwd   :828-850   -> [out, softmax_lse, p, rng_state]
  bwd         <- mha_bwd          :1251-1271 -> [dq, dk, dv, softmax_d]
  varlen_bwd  <- mha_varlen_bwd   :1063-1087 -> [dq, dk, dv, softmax_d]
  fwd_kvcache <- mha_fwd_kvcache  :356-377   -> [out, softmax_lse]

so the reference's own Python layer (flash_attn_npu_v2/interface_arch22.py)
can import it in place of the NPU extension. p (the attention probabilities)
and rng_state are empty: there is no dropout. Caller-given out / dq / dk / dv
receive the results."""
import torch

from fa_mi355x import ops


def _empty(like):
    return torch.empty((0,), dtype=torch.float32, device=like.device)


def _into(dst, src):
    if dst is None:
        return src
    dst.copy_(src)
    return dst


def fwd(q, k, v, out_, alibi_slopes, p_dropout, softmax_scale, is_causal, window_size_left, window_size_right,
        softcap, return_softmax, gen_=None):
    out, lse = ops.fwd(q, k, v, alibi_slopes, float(p_dropout), float(softmax_scale), bool(is_causal),
                       int(window_size_left), int(window_size_right), float(softcap))
    return [_into(out_, out), lse, _empty(q), _empty(q)]


def varlen_fwd(q, k, v, out_, cu_seqlens_q, cu_seqlens_k, seqused_k, leftpad_k, block_table, alibi_slopes,
               max_seqlen_q, max_seqlen_k, p_dropout, softmax_scale, zero_tensors, is_causal, window_size_left,
               window_size_right, softcap, return_softmax, gen_=None):
    if leftpad_k is not None:
        raise RuntimeError("leftpad_k is not supported by varlen_fwd")
    out, lse = ops.varlen_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, block_table, alibi_slopes,
                              int(max_seqlen_q), int(max_seqlen_k), float(p_dropout), float(softmax_scale),
                              bool(is_causal), int(window_size_left), int(window_size_right), float(softcap))
    return [_into(out_, out), lse, _empty(q), _empty(q)]


def bwd(dout, q, k, v, out, softmax_lse, dq_, dk_, dv_, alibi_slopes, p_dropout, softmax_scale, is_causal,
        window_size_left, window_size_right, softcap, deterministic, gen_=None, rng_state=None):
    dq, dk, dv, sd = ops.bwd(dout, q, k, v, out, softmax_lse, alibi_slopes, float(p_dropout), float(softmax_scale),
                             bool(is_causal), int(window_size_left), int(window_size_right), float(softcap),
                             bool(deterministic))
    return [_into(dq_, dq), _into(dk_, dk), _into(dv_, dv), sd]


def varlen_bwd(dout, q, k, v, out, softmax_lse, dq_, dk_, dv_, cu_seqlens_q, cu_seqlens_k, alibi_slopes,
               max_seqlen_q, max_seqlen_k, p_dropout, softmax_scale, zero_tensors, is_causal, window_size_left,
               window_size_right, softcap, deterministic, gen_=None, rng_state=None):
    dq, dk, dv, sd = ops.varlen_bwd(dout, q, k, v, out, softmax_lse, cu_seqlens_q, cu_seqlens_k, alibi_slopes,
                                    int(max_seqlen_q), int(max_seqlen_k), float(p_dropout), float(softmax_scale),
                                    bool(is_causal), int(window_size_left), int(window_size_right), float(softcap),
                                    bool(deterministic))
    return [_into(dq_, dq), _into(dk_, dk), _into(dv_, dv), sd]


def fwd_kvcache(q, kcache, vcache, k_, v_, seqlens_k, rotary_cos, rotary_sin, cache_batch_idx, leftpad_k,
                block_table, alibi_slopes, out_, softmax_scale, is_causal, window_size_left, window_size_right,
                softcap, is_rotary_interleaved, num_splits):
    out, lse = ops.fwd_kvcache(q, kcache, vcache, k_, v_, seqlens_k, rotary_cos, rotary_sin, cache_batch_idx,
                               leftpad_k, block_table, alibi_slopes, float(softmax_scale), bool(is_causal),
                               int(window_size_left), int(window_size_right), float(softcap),
                               bool(is_rotary_interleaved), int(num_splits))
    return [_into(out_, out), lse]
