"""get_scheduler_metadata on the host: the descriptor header round-trips, the
workspace comes from the library's planner, and a call that differs in any
checked field is refused (flash_attn_npu_v3/interface_arch22.py:1098-1138 and
tests/test_flash_attn_npu_v3_metadata.py of the reference)."""
import pytest
import torch

from flash_attn_npu_v3 import interface as v3


def _md(**kw):
    args = dict(batch_size=3, max_seqlen_q=64, max_seqlen_k=4096, num_heads_q=16, num_heads_kv=4, headdim=128,
                cache_seqlens=torch.zeros(3, dtype=torch.int32), causal=True)
    args.update(kw)
    return v3.get_scheduler_metadata(**args)


def _call(**kw):
    d = dict(batch=3, max_seqlen_q=64, max_seqlen_k=4096, nheads=16, nheads_k=4, headdim=128, headdim_v=128,
             dtype=torch.bfloat16, causal=True, window_size=(-1, -1), attention_chunk=0, softcap=0.0, num_splits=1,
             page_size=0, varlen_q=False)
    d.update(kw)
    return v3._describe(**d)


def test_header_round_trip_and_workspace():
    md = _md(page_size=256, num_splits=3)
    d = md._fa_metadata
    assert v3._read_header(md) == d
    assert md.numel() == 256 + d["workspace_bytes"] and d["workspace_bytes"] > 0
    assert d["num_splits"] == 3 and d["page_size"] == 256 and d["window_right"] == 0


def test_matching_call_takes_workspace_and_splits():
    md = _md(num_splits=4)
    ws, ns = v3._metadata_for(md, _call(num_splits=1), torch.device("cpu"))
    assert ns == 4 and ws.numel() == md.numel() - 256 and ws.data_ptr() == md.data_ptr() + 256
    # shorter queries than planned are fine
    v3._metadata_for(md, _call(max_seqlen_q=10), torch.device("cpu"))


@pytest.mark.parametrize("change", [dict(batch=4), dict(nheads=32), dict(nheads_k=8), dict(headdim=64, headdim_v=64),
                                    dict(dtype=torch.float16), dict(causal=False), dict(window_size=(100, 0)),
                                    dict(attention_chunk=64), dict(softcap=30.0), dict(page_size=64),
                                    dict(varlen_q=True), dict(max_seqlen_q=65)])
def test_mismatch_raises(change):
    md = _md()
    with pytest.raises(RuntimeError, match="different call"):
        v3._metadata_for(md, _call(**change), torch.device("cpu"))


def test_copy_is_checked_through_its_header():
    md = _md()
    cp = md.clone()  # the Python-side descriptor does not survive the copy
    assert getattr(cp, "_fa_metadata", None) is None
    v3._metadata_for(cp, _call(), torch.device("cpu"))
    with pytest.raises(RuntimeError, match="different call"):
        v3._metadata_for(cp, _call(batch=2), torch.device("cpu"))
    bad = torch.zeros(512, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="does not come from"):
        v3._metadata_for(bad, _call(), torch.device("cpu"))
    with pytest.raises(RuntimeError, match="uint8 tensor"):
        v3._metadata_for(torch.zeros(64, dtype=torch.int32), _call(), torch.device("cpu"))


@pytest.mark.parametrize("B,H,Hk,D,maxq,page,splits", [
    (64, 16, 4, 128, 64, 0, 0), (3, 16, 4, 128, 64, 0, 0), (3, 16, 4, 128, 64, 256, 0), (2, 32, 8, 256, 300, 0, 0),
    (5, 8, 8, 64, 40, 0, 3), (1, 40, 8, 111, 90, 0, 0)])
def test_workspace_covers_every_shorter_call(B, H, Hk, D, maxq, page, splits):
    """A call of any query length up to max_seqlen_q, packed or not, fits the
    planned workspace, also where a shorter call switches to the decode kernel
    or to an automatic split over the key range (which need more scratch than
    the call at max_seqlen_q)."""
    md = v3.get_scheduler_metadata(B, maxq, 4096, H, Hk, D, cache_seqlens=torch.zeros(B, dtype=torch.int32),
                                   page_size=page or None, num_splits=splits, causal=True)
    d = md._fa_metadata
    room = md.numel() - 256
    for sq in range(1, maxq + 1):
        for no_pack in (0, 1):
            assert v3._workspace_at(d, sq, no_pack) <= room, (sq, no_pack)


def test_workspace_short_decode_call_direct():
    """The library planner itself, for a decode-sized call (Sq = 4) under
    metadata planned at Sq = 64: the decode's partials fit."""
    from fa_mi355x import capi
    B, H, Hk, D = 64, 16, 4, 128
    md = v3.get_scheduler_metadata(B, 64, 4096, H, Hk, D, cache_seqlens=torch.zeros(B, dtype=torch.int32),
                                   causal=True)
    dummy = 1 << 20
    p = capi.new_params(dtype=1, batch=B, seqlen_q=4, nheads=H, nheads_k=Hk, headdim=D, headdim_v=D, q=dummy,
                        q_batch_stride=4 * H * D, q_row_stride=H * D, q_head_stride=D, k=dummy,
                        k_batch_stride=4096 * Hk * D, k_row_stride=Hk * D, k_head_stride=D, v=dummy,
                        v_batch_stride=4096 * Hk * D, v_row_stride=Hk * D, v_head_stride=D, out=dummy,
                        out_batch_stride=4 * H * D, out_row_stride=H * D, out_head_stride=D, softmax_lse=dummy,
                        cache_seqlens=dummy, seqlen_k=4096, batch_cache=B, softmax_scale=1.0, is_causal=1)
    st, need = capi.workspace_size(p, capi.FA_KIND_KVCACHE)
    assert st == capi.FA_OK and need > 1 << 20
    assert need <= md.numel() - 256


def test_workspace_forced_split_qv_decode_direct():
    """A forced split count sends decode-sized calls to the split prefill path,
    but a kvcache call with qv stays on the decode kernel (only it forms the qv
    term) and keeps the decode's partials: metadata planned with num_splits=3
    holds them (the library planner itself, asked for that call)."""
    from fa_mi355x import capi
    B, H, Hk, D, Sq = 1, 16, 4, 128, 4
    md = v3.get_scheduler_metadata(B, Sq, 4096, H, Hk, D, cache_seqlens=torch.zeros(B, dtype=torch.int32),
                                   num_splits=3, causal=True)
    dummy = 1 << 20
    kw = dict(dtype=1, batch=B, seqlen_q=Sq, nheads=H, nheads_k=Hk, headdim=D, headdim_v=D, q=dummy,
              q_batch_stride=Sq * H * D, q_row_stride=H * D, q_head_stride=D, k=dummy,
              k_batch_stride=4096 * Hk * D, k_row_stride=Hk * D, k_head_stride=D, v=dummy,
              v_batch_stride=4096 * Hk * D, v_row_stride=Hk * D, v_head_stride=D, out=dummy,
              out_batch_stride=Sq * H * D, out_row_stride=H * D, out_head_stride=D, softmax_lse=dummy,
              cache_seqlens=dummy, seqlen_k=4096, batch_cache=B, softmax_scale=1.0, is_causal=1, num_splits=3)
    st, plain = capi.workspace_size(capi.new_params(**kw), capi.FA_KIND_KVCACHE)
    st2, with_qv = capi.workspace_size(capi.new_params(**kw, qv=dummy, qv_batch_stride=Sq * H * D,
                                                       qv_row_stride=H * D, qv_head_stride=D), capi.FA_KIND_KVCACHE)
    assert st == capi.FA_OK and st2 == capi.FA_OK
    assert with_qv > plain  # the decode plan's partials, larger than the split prefill's here
    assert with_qv <= md.numel() - 256
