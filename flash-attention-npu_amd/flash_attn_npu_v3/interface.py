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


# ---- scheduler metadata -------------------------------------------------------------------------
# get_scheduler_metadata (interface_arch22.py:1098-1138 of the reference) returns
# the plan of a later call: here a uint8 device buffer of a 256-byte header
# (the problem descriptor below, int32) followed by the call's workspace, sized
# by the library's planner (fa_fwd_workspace_size). A v3 call given the buffer
# checks that it describes the call (raising otherwise), takes the split count
# from it (as the reference takes its split plan from the metadata,
# flash_api.cpp:249-269) and runs on its workspace, so it allocates no scratch.
# The per-sequence split itself is still decided on the device from
# cache_seqlens, so the results equal those of the same call without metadata.
# The buffer is the call's scratch: calls that use one buffer must not overlap
# (one stream, or ordered streams).
_MD_TAG = 0x46414D44  # "FAMD"
_MD_VERSION = 1
_MD_HEADER = 256
_MD_FIELDS = ("batch", "max_seqlen_q", "max_seqlen_k", "nheads", "nheads_k", "headdim", "headdim_v", "dtype",
              "causal", "window_left", "window_right", "attention_chunk", "softcap", "num_splits", "page_size",
              "varlen_q", "workspace_bytes")
# fields a call must match; max_seqlen_q bounds the call's query length
_MD_CHECKED = ("batch", "nheads", "nheads_k", "headdim", "headdim_v", "dtype", "causal", "window_left",
               "window_right", "attention_chunk", "softcap", "page_size", "varlen_q")


def _dtype_code(dt):
    codes = {torch.float16: 0, torch.bfloat16: 1, torch.float8_e4m3fn: 3}
    if dt not in codes:
        raise RuntimeError("FlashAttention only support fp16 and bf16 data type")
    return codes[dt]


def _describe(batch, max_seqlen_q, max_seqlen_k, nheads, nheads_k, headdim, headdim_v, dtype, causal, window_size,
              attention_chunk, softcap, num_splits, page_size, varlen_q):
    wl = -1 if window_size[0] < 0 else int(window_size[0])
    wr = -1 if window_size[1] < 0 else int(window_size[1])
    if causal:
        wr = 0
    if dtype in (torch.float16, torch.bfloat16):
        # the head dims the kernels run at: 16-bit rows are zero-padded to a
        # multiple of 8 (_needs_pad), so a call and its padded form share a plan
        headdim, headdim_v = -(-int(headdim) // 8) * 8, -(-int(headdim_v) // 8) * 8
    return dict(batch=int(batch), max_seqlen_q=int(max_seqlen_q), max_seqlen_k=int(max_seqlen_k), nheads=int(nheads),
                nheads_k=int(nheads_k), headdim=int(headdim), headdim_v=int(headdim_v), dtype=_dtype_code(dtype),
                causal=int(bool(causal)), window_left=wl, window_right=wr, attention_chunk=int(attention_chunk),
                softcap=int(bool(softcap)), num_splits=int(num_splits), page_size=int(page_size or 0),
                varlen_q=int(bool(varlen_q)), workspace_bytes=0)


def _plan_workspace(d):
    """Largest workspace any call of this description needs, from the
    library's own planner: every query length up to max_seqlen_q, packed and
    unpacked GQA, and the kvcache call with rotary included.

    Within each kernel regime the planner's need grows with the query length
    (decode: <= 16 packed rows per kv head, its rotated-q copy grows; prefill
    split over the key range while batch x kv heads x row tiles leave CUs
    idle, its partial rows grow; prefill unsplit: no partials), and the
    regimes follow one another in that order as the query length grows. So
    the largest need is at the right end of a regime: the last decode length,
    the last split length (found by bisection) or max_seqlen_q."""
    maxq = max(d["max_seqlen_q"], 1)
    g = d["nheads"] // max(d["nheads_k"], 1)
    need = None
    for no_pack in (0, 1):
        ge = 1 if no_pack else max(g, 1)
        need_at = lambda sq: _workspace_at(d, sq, no_pack)  # noqa: E731
        base = need_at(maxq)
        lengths = {1, maxq, min(maxq, max(1, 16 // ge))}
        # the last length whose plan has partial rows (decode or split prefill);
        # `bare` is a plan without any: unsplit prefill (17 unpacked rows)
        bare = _workspace_at(dict(d, num_splits=1), 17, 1)
        if need_at(1) > bare:
            lo, hi = 1, maxq
            while lo < hi:
                mid = (lo + hi + 1) // 2
                if need_at(mid) > bare:
                    lo = mid
                else:
                    hi = mid - 1
            lengths.add(lo)
        for sq in lengths:
            n = base if sq == maxq else need_at(sq)
            need = n if need is None else max(need, n)
    return need


def _workspace_at(d, Sq, no_pack):
    """The planner's workspace for the calls of description `d` at query
    length Sq (the largest over the call kinds the description allows)."""
    from fa_mi355x import capi
    B, Sk, H, Hk, D = d["batch"], max(d["max_seqlen_k"], 1), d["nheads"], d["nheads_k"], \
        -(-d["headdim"] // 8) * 8
    dummy = 1 << 20  # aligned stand-in addresses: the planner never dereferences them
    common = dict(dtype=d["dtype"], batch=B, seqlen_q=Sq, nheads=H, nheads_k=Hk, headdim=D, headdim_v=D,
                  q=dummy, q_batch_stride=Sq * H * D, q_row_stride=H * D, q_head_stride=D,
                  k=dummy, k_batch_stride=Sk * Hk * D, k_row_stride=Hk * D, k_head_stride=D,
                  v=dummy, v_batch_stride=Sk * Hk * D, v_row_stride=Hk * D, v_head_stride=D,
                  out=dummy, out_batch_stride=Sq * H * D, out_row_stride=H * D, out_head_stride=D,
                  softmax_lse=dummy, softmax_scale=1.0, is_causal=d["causal"],
                  window_size_left=d["window_left"], window_size_right=d["window_right"],
                  attention_chunk=d["attention_chunk"], softcap=1.0 if d["softcap"] else 0.0,
                  num_splits=d["num_splits"], no_pack_gqa=no_pack)
    if d["varlen_q"]:
        common.update(cu_seqlens_q=dummy, total_q=B * Sq)
    cands = []
    page = d["page_size"]
    kv = dict(cache_seqlens=dummy, seqlen_k=Sk, batch_cache=B)
    if page:
        nper = (Sk + page - 1) // page
        kv = dict(cache_seqlens=dummy, block_table=dummy, block_table_batch_stride=nper, max_blocks_per_seq=nper,
                  block_table_rows=B, page_block_size=page, batch_cache=B * nper, seqlen_k=0)
    cands.append((capi.FA_KIND_KVCACHE, dict(common, **kv)))
    if d["dtype"] != 3 and D >= 16:
        cands.append((capi.FA_KIND_KVCACHE, dict(common, **kv, k_new=dummy, v_new=dummy, seqlen_new=1,
                                                 knew_batch_stride=Hk * D, knew_row_stride=Hk * D,
                                                 knew_head_stride=D, vnew_batch_stride=Hk * D,
                                                 vnew_row_stride=Hk * D, vnew_head_stride=D, rotary_cos=dummy,
                                                 rotary_sin=dummy, rotary_dim=16, seqlen_ro=Sk)))
    if d["dtype"] != 3:
        # a kvcache call with qv keeps the decode kernel's plan whatever num_splits says
        cands.append((capi.FA_KIND_KVCACHE, dict(common, **kv, qv=dummy, qv_batch_stride=Sq * H * D,
                                                 qv_row_stride=H * D, qv_head_stride=D)))
    if not page:
        cands.append((capi.FA_KIND_DENSE, dict(common, seqlen_k=Sk, batch_cache=B)))
    cands.append((capi.FA_KIND_VARLEN, dict(common, cu_seqlens_q=dummy, cu_seqlens_k=dummy, total_q=B * Sq,
                                            seqlen_k=Sk, batch_cache=B)))
    need = None
    for kind, kw in cands:
        st, n = capi.workspace_size(capi.new_params(**kw), kind)
        if st == capi.FA_OK:
            need = n if need is None else max(need, n)
    if need is None:
        raise RuntimeError("get_scheduler_metadata: " + capi.last_error())
    return need


def _header_tensor(d):
    vals = [_MD_TAG, _MD_VERSION] + [d[f] for f in _MD_FIELDS]
    h = torch.zeros(_MD_HEADER // 4, dtype=torch.int32)
    h[:len(vals)] = torch.tensor(vals, dtype=torch.int64).to(torch.int32)
    return h.view(torch.uint8)


def _read_header(md):
    h = md[:_MD_HEADER].cpu().view(torch.int32).tolist()
    if h[0] != _MD_TAG or h[1] != _MD_VERSION:
        raise RuntimeError("scheduler_metadata does not come from get_scheduler_metadata")
    return dict(zip(_MD_FIELDS, h[2:2 + len(_MD_FIELDS)]))


def _metadata_for(scheduler_metadata, call, device):
    """The workspace region of `scheduler_metadata` and its split count, after
    checking that it describes `call`; (None, None) without metadata."""
    md = scheduler_metadata
    if md is None:
        return None, None
    if not isinstance(md, torch.Tensor) or md.dtype != torch.uint8 or md.dim() != 1 or not md.is_contiguous() \
            or md.numel() < _MD_HEADER:
        raise RuntimeError("scheduler_metadata must be the uint8 tensor get_scheduler_metadata returns")
    if md.device != device:
        raise RuntimeError("scheduler_metadata must be on the same device as q")
    d = getattr(md, "_fa_metadata", None)
    if d is None:  # a copy: read the header back (this synchronises, as the reference does)
        d = _read_header(md)
    bad = [f"{f} {d[f]} != {call[f]}" for f in _MD_CHECKED if d[f] != call[f]]
    if call["max_seqlen_q"] > d["max_seqlen_q"]:
        bad.append(f"max_seqlen_q {call['max_seqlen_q']} > {d['max_seqlen_q']}")
    if bad:
        raise RuntimeError("scheduler_metadata was made for a different call: " + ", ".join(bad))
    return md[_MD_HEADER:], d["num_splits"]


def _cu_from_lengths(lengths):
    z = torch.zeros((1,), dtype=torch.int32, device=lengths.device)
    return torch.cat([z, torch.cumsum(lengths, 0, dtype=torch.int32)])


def _pack(pack_gqa):
    return None if pack_gqa is None else bool(pack_gqa)


def _needs_pad(x):
    """16-bit inputs whose head dim is not a multiple of 8: the kernels load
    16-byte chunks of a head row, so such rows are zero-padded to the next
    multiple of 8 (zeros add nothing to q.k and give zero output columns,
    which are sliced off). The reference v3 accepts any head dim <= 256
    (csrc/arch22/flash_attn_npu_v3/flash_api.cpp:201-218); FP8 keeps its own
    multiple-of-16 rule."""
    return x is not None and x.shape[-1] % 8 != 0 and x.dtype in (torch.float16, torch.bfloat16)


def _pad_last(x, width):
    return x if x is None or x.shape[-1] == width else torch.nn.functional.pad(x, [0, width - x.shape[-1]])


def _padded_head(attn, q, k, v, return_lse):
    """attn(q, k, v) on rows zero-padded to a multiple of 8 (differentiable:
    the gradient of the padding is the slice), output sliced back."""
    dv = v.shape[-1]
    w = -(-max(q.shape[-1], dv) // 8) * 8
    res = attn(_pad_last(q, w), _pad_last(k, w), _pad_last(v, w))
    if return_lse:
        return res[0][..., :dv], res[1]
    return res[..., :dv]


def _qv_by_concat(attn, q, k, v, qv, return_lse):
    """FlashAttention-3's qv for the prefill kernels: scores = q.k + qv.v is
    one attention over the head dims of q and qv concatenated, against k and
    v concatenated; v is zero-padded to that width and the padding sliced off
    the output. (The decode kernel takes qv directly.)"""
    if qv.dtype != q.dtype or qv.shape[:-1] != q.shape[:-1] or qv.shape[-1] != v.shape[-1]:
        raise RuntimeError("qv must have the dtype of q and shape q.shape[:-1] + (headdim_v,)")
    dv = v.shape[-1]
    q2 = torch.cat([q, qv], dim=-1)
    k2 = torch.cat([k, v], dim=-1)
    v2 = torch.cat([v, torch.zeros_like(k)], dim=-1)
    res = _padded_head(attn, q2, k2, v2, return_lse) if _needs_pad(q2) else attn(q2, k2, v2)
    if return_lse:
        return res[0][..., :dv], res[1]
    return res[..., :dv]


class FlashAttnFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, softmax_scale, causal, qv=None, q_descale=None, k_descale=None, v_descale=None,
                window_size=(-1, -1), attention_chunk=0, softcap=0.0, num_splits=1, pack_gqa=None,
                deterministic=False, sm_margin=0, return_softmax=False, scheduler_metadata=None):
        if softmax_scale is None:
            softmax_scale = (q.shape[-1] + (qv.shape[-1] if qv is not None else 0)) ** (-0.5)
        call = _describe(q.shape[0], q.shape[1], k.shape[1], q.shape[2], k.shape[2], q.shape[3], v.shape[3], q.dtype,
                         causal, window_size, attention_chunk, softcap, num_splits, 0, False)
        ws, md_splits = _metadata_for(scheduler_metadata, call, q.device)
        if md_splits is not None:
            num_splits = md_splits
        q, k, v = [maybe_contiguous(x) for x in (q, k, v)]
        out, softmax_lse = ops.fwd(q, k, v, None, 0.0, float(softmax_scale), bool(causal), int(window_size[0]),
                                   int(window_size[1]), float(softcap), int(attention_chunk), q_descale, k_descale,
                                   v_descale, int(num_splits), ws, _pack(pack_gqa))
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
        _reject(seqused_q=seqused_q)
        if softmax_scale is None:
            softmax_scale = (q.shape[-1] + (qv.shape[-1] if qv is not None else 0)) ** (-0.5)
        call = _describe(cu_seqlens_q.numel() - 1, max_seqlen_q, max_seqlen_k, q.shape[1], k.shape[1], q.shape[2],
                         v.shape[2], q.dtype, causal, window_size, attention_chunk, softcap, num_splits, 0, True)
        ws, md_splits = _metadata_for(scheduler_metadata, call, q.device)
        if md_splits is not None:
            num_splits = md_splits
        q, k, v = [maybe_contiguous(x) for x in (q, k, v)]
        out, softmax_lse = ops.varlen_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_k, None, None,
                                          int(max_seqlen_q), int(max_seqlen_k), 0.0, float(softmax_scale),
                                          bool(causal), int(window_size[0]), int(window_size[1]), float(softcap),
                                          int(attention_chunk), q_descale, k_descale, v_descale, int(num_splits), ws,
                                          _pack(pack_gqa))
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
    qv (batch_size, seqlen, nheads, headdim_v) adds qv . v to the scores (the
    default scale is then (headdim + headdim_v) ** -0.5). pack_gqa = False
    gives each query head its own row tiles (the same results to rounding).
    Returns out, or (out, softmax_lse (batch, nheads, seqlen)) when return_attn_probs."""
    if qv is not None:
        if softmax_scale is None:
            softmax_scale = (q.shape[-1] + qv.shape[-1]) ** (-0.5)
        return _qv_by_concat(lambda q2, k2, v2: FlashAttnFunc.apply(
            q2, k2, v2, softmax_scale, causal, None, q_descale, k_descale, v_descale, window_size, attention_chunk,
            softcap, num_splits, pack_gqa, deterministic, sm_margin, return_attn_probs, scheduler_metadata),
            q, k, v, qv, return_attn_probs)
    if _needs_pad(q):
        if softmax_scale is None:
            softmax_scale = q.shape[-1] ** (-0.5)
        return _padded_head(lambda q2, k2, v2: FlashAttnFunc.apply(
            q2, k2, v2, softmax_scale, causal, None, q_descale, k_descale, v_descale, window_size, attention_chunk,
            softcap, num_splits, pack_gqa, deterministic, sm_margin, return_attn_probs,
            scheduler_metadata), q, k, v, return_attn_probs)
    return FlashAttnFunc.apply(q, k, v, softmax_scale, causal, qv, q_descale, k_descale, v_descale, window_size,
                               attention_chunk, softcap, num_splits, pack_gqa, deterministic, sm_margin,
                               return_attn_probs, scheduler_metadata)


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, seqused_q=None,
                           seqused_k=None, softmax_scale=None, causal=False, qv=None, q_descale=None, k_descale=None,
                           v_descale=None, window_size=(-1, -1), attention_chunk=0, softcap=0.0, num_splits=1,
                           pack_gqa=None, deterministic=False, sm_margin=0, return_attn_probs=False,
                           scheduler_metadata=None):
    """q: (total_q, nheads, headdim); k, v: (total_k, nheads_k, headdim).
    softmax_lse is (nheads, total_q). qv (total_q, nheads, headdim_v) and
    pack_gqa as in flash_attn_func."""
    if qv is not None:
        if softmax_scale is None:
            softmax_scale = (q.shape[-1] + qv.shape[-1]) ** (-0.5)
        return _qv_by_concat(lambda q2, k2, v2: FlashAttnVarlenFunc.apply(
            q2, k2, v2, cu_seqlens_q, cu_seqlens_k, seqused_q, seqused_k, max_seqlen_q, max_seqlen_k,
            softmax_scale, causal, None, q_descale, k_descale, v_descale, window_size, attention_chunk, softcap,
            num_splits, pack_gqa, deterministic, sm_margin, return_attn_probs, scheduler_metadata),
            q, k, v, qv, return_attn_probs)
    if _needs_pad(q):
        if softmax_scale is None:
            softmax_scale = q.shape[-1] ** (-0.5)
        return _padded_head(lambda q2, k2, v2: FlashAttnVarlenFunc.apply(
            q2, k2, v2, cu_seqlens_q, cu_seqlens_k, seqused_q, seqused_k, max_seqlen_q, max_seqlen_k,
            softmax_scale, causal, None, q_descale, k_descale, v_descale, window_size, attention_chunk, softcap,
            num_splits, pack_gqa, deterministic, sm_margin, return_attn_probs,
            scheduler_metadata), q, k, v, return_attn_probs)
    return FlashAttnVarlenFunc.apply(q, k, v, cu_seqlens_q, cu_seqlens_k, seqused_q, seqused_k, max_seqlen_q,
                                     max_seqlen_k, softmax_scale, causal, qv, q_descale, k_descale, v_descale,
                                     window_size, attention_chunk, softcap, num_splits, pack_gqa, deterministic,
                                     sm_margin, return_attn_probs, scheduler_metadata)


def flash_attn_combine(out_partial, lse_partial, out=None, out_dtype=None):
    """Merge split-KV partials: out_partial (num_splits, ..., headdim_v) fp32 and
    lse_partial (num_splits, ...) fp32 -> (out, lse) with
    lse = log sum_s exp(lse_s) and out = sum_s exp(lse_s - lse) out_s. With
    `out` given, the merged rows are written into it (fp32, bf16 or fp16)."""
    if out is not None:
        return out, ops.fwd_combine_out(out_partial, lse_partial, out)
    return ops.fwd_combine(out_partial, lse_partial, out_dtype)


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
    if softmax_scale is None:
        softmax_scale = (q.shape[-1] + (qv.shape[-1] if qv is not None else 0)) ** (-0.5)
    batch = q.shape[0] if cu_seqlens_q is None else cu_seqlens_q.numel() - 1
    if cache_seqlens is not None and isinstance(cache_seqlens, int):
        cache_seqlens = torch.full((batch,), cache_seqlens, dtype=torch.int32, device=k_cache.device)
    cache_seqlens = maybe_contiguous(cache_seqlens)
    paged = page_table is not None
    packed = cu_seqlens_q is not None and not paged and k_cache.dim() == 3
    sq = int(max_seqlen_q) if cu_seqlens_q is not None and max_seqlen_q is not None else q.shape[-3]
    cap = k_cache.shape[0] if packed else (page_table.shape[1] * k_cache.shape[1] if paged else k_cache.shape[1])
    call = _describe(batch, sq, cap, q.shape[-2], k_cache.shape[-2], q.shape[-1], v_cache.shape[-1], q.dtype, causal,
                     window_size, attention_chunk, softcap, num_splits, k_cache.shape[1] if paged else 0,
                     cu_seqlens_q is not None)
    ws, md_splits = _metadata_for(scheduler_metadata, call, q.device)
    if md_splits is not None:
        num_splits = md_splits
    pad_d = _needs_pad(q)
    if pad_d:
        # head dims not a multiple of 8 (_needs_pad): the call runs on
        # zero-padded copies of q, k / v, qv and the caches; the caches'
        # real columns are copied back after an append, and out is sliced
        d_og, dv_og = q.shape[-1], v_cache.shape[-1]
        w = -(-max(d_og, dv_og) // 8) * 8
        kc_user, vc_user = k_cache, v_cache
        k_cache, v_cache = _pad_last(k_cache, w), _pad_last(v_cache, w)
        q, k, v, qv = (_pad_last(x, w) for x in (q, k, v, qv))
    q, k, v = [maybe_contiguous(x) for x in (q, k, v)]
    if cu_seqlens_q is not None and max_seqlen_q is None:
        raise RuntimeError("max_seqlen_q is required with cu_seqlens_q")
    if cu_seqlens_q is not None and page_table is None and k_cache.dim() == 3:
        # varlen (TND) queries against a packed (total_k, nheads_k, headdim)
        # cache indexed by the prefix sums of cache_seqlens
        # (csrc/arch22/flash_attn_npu_v3/flash_api.cpp:431-441 in the reference)
        _reject(k=k, v=v, rotary_cos=rotary_cos, cache_batch_idx=cache_batch_idx, cache_leftpad=cache_leftpad,
                cu_seqlens_k_new=cu_seqlens_k_new, qv=qv)
        if cache_seqlens is None:
            raise RuntimeError("cache_seqlens is required with cu_seqlens_q")
        cu_k = _cu_from_lengths(cache_seqlens)
        out, softmax_lse = ops.varlen_fwd(q, k_cache, v_cache, cu_seqlens_q, cu_k, cache_seqlens, None, None,
                                          int(max_seqlen_q), int(k_cache.shape[0]), 0.0, float(softmax_scale),
                                          bool(causal), int(window_size[0]), int(window_size[1]), float(softcap),
                                          int(attention_chunk), q_descale, k_descale, v_descale, int(num_splits), ws,
                                          _pack(pack_gqa))
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
                                              v_descale, ws, maybe_contiguous(qv), _pack(pack_gqa))
    if pad_d:
        out = out[..., :dv_og]
        if k is not None:
            kc_user.copy_(k_cache[..., :d_og])
            vc_user.copy_(v_cache[..., :dv_og])
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
    """The plan of a later flash_attn_with_kvcache / flash_attn_func /
    flash_attn_varlen_func call (same keywords as the reference,
    interface_arch22.py:1098-1138): a uint8 tensor on the device of
    cache_seqlens holding the call's descriptor and its workspace (see the
    scheduler-metadata notes above). A call given it raises when it describes
    a different problem."""
    if headdim_v is None:
        headdim_v = headdim
    if num_splits < 0:
        raise RuntimeError("num_splits must be >= 0")
    d = _describe(batch_size, max_seqlen_q, max_seqlen_k, num_heads_q, num_heads_kv, headdim, headdim_v, qkv_dtype,
                  causal, window_size, attention_chunk, has_softcap, num_splits, page_size, cu_seqlens_q is not None)
    d["workspace_bytes"] = _plan_workspace(d)
    md = torch.empty((_MD_HEADER + d["workspace_bytes"],), dtype=torch.uint8, device=cache_seqlens.device)
    md[:_MD_HEADER].copy_(_header_tensor(d))
    md._fa_metadata = d
    return md
