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
