"""Meta (fake) implementations of the fa_mi355x operators, so the ops trace
under torch.compile. Output shapes follow the reference fakes
(flash_attn_npu_v3/interface_arch22.py:157-259, flash_attn_npu_v2/
interface_arch22.py:79-106,178-199): out like q, LSE (B, H, Sq) fp32, or
(H, total_q) for the varlen layout. FP8 (e4m3) inputs give a bf16 out."""
import torch


def _out_like(q):
    if q.dtype == torch.float8_e4m3fn:
        return torch.empty_like(q, dtype=torch.bfloat16)
    return torch.empty_like(q)


@torch.library.register_fake("fa_mi355x::fwd_kvcache")
def _fwd_kvcache_fake(q, k_cache, v_cache, k, v, seqlens_k, rotary_cos, rotary_sin, cache_batch_idx, leftpad_k,
                      block_table, alibi_slopes, softmax_scale, is_causal, window_size_left, window_size_right,
                      softcap, is_rotary_interleaved, num_splits):
    b, sq, h, _ = q.shape
    return _out_like(q), q.new_empty((b, h, sq), dtype=torch.float32)


@torch.library.register_fake("fa_mi355x::fwd_kvcache_v3")
def _fwd_kvcache_v3_fake(q, k_cache, v_cache, k, v, seqlens_k, rotary_cos, rotary_sin, cache_batch_idx, leftpad_k,
                         block_table, alibi_slopes, cu_seqlens_q, cu_seqlens_k_new, max_seqlen_q, rotary_seqlens,
                         softmax_scale, is_causal, window_size_left, window_size_right, attention_chunk, softcap,
                         is_rotary_interleaved, num_splits, q_descale=None, k_descale=None, v_descale=None,
                         workspace=None, qv=None, pack_gqa=None):
    if cu_seqlens_q is not None:
        t, h, _ = q.shape
        return _out_like(q), q.new_empty((h, t), dtype=torch.float32)
    b, sq, h, _ = q.shape
    return _out_like(q), q.new_empty((b, h, sq), dtype=torch.float32)


@torch.library.register_fake("fa_mi355x::fwd")
def _fwd_fake(q, k, v, alibi_slopes, p_dropout, softmax_scale, is_causal, window_size_left, window_size_right,
              softcap, attention_chunk=0, q_descale=None, k_descale=None, v_descale=None, num_splits=0,
              workspace=None, pack_gqa=None):
    b, sq, h, _ = q.shape
    return _out_like(q), q.new_empty((b, h, sq), dtype=torch.float32)


@torch.library.register_fake("fa_mi355x::varlen_fwd")
def _varlen_fwd_fake(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, block_table, alibi_slopes, max_seqlen_q, max_seqlen_k,
                     p_dropout, softmax_scale, is_causal, window_size_left, window_size_right, softcap,
                     attention_chunk=0, q_descale=None, k_descale=None, v_descale=None, num_splits=0,
                     workspace=None, pack_gqa=None):
    t, h, _ = q.shape
    return _out_like(q), q.new_empty((h, t), dtype=torch.float32)


@torch.library.register_fake("fa_mi355x::fwd_combine")
def _fwd_combine_fake(out_partial, lse_partial, out_dtype):
    dt = out_dtype if out_dtype is not None else torch.float32
    return out_partial.new_empty(out_partial.shape[1:], dtype=dt), lse_partial.new_empty(lse_partial.shape[1:])


@torch.library.register_fake("fa_mi355x::fwd_combine_out")
def _fwd_combine_out_fake(out_partial, lse_partial, out):
    return lse_partial.new_empty(lse_partial.shape[1:])


@torch.library.register_fake("fa_mi355x::bwd")
def _bwd_fake(dout, q, k, v, out, softmax_lse, alibi_slopes, p_dropout, softmax_scale, is_causal, window_size_left,
              window_size_right, softcap, deterministic, attention_chunk=0):
    b, sq, h, _ = q.shape
    return (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
            q.new_empty((b, h, sq), dtype=torch.float32))


@torch.library.register_fake("fa_mi355x::varlen_bwd")
def _varlen_bwd_fake(dout, q, k, v, out, softmax_lse, cu_seqlens_q, cu_seqlens_k, alibi_slopes, max_seqlen_q,
                     max_seqlen_k, p_dropout, softmax_scale, is_causal, window_size_left, window_size_right, softcap,
                     deterministic, attention_chunk=0):
    t, h, _ = q.shape
    return (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
            q.new_empty((h, t), dtype=torch.float32))
