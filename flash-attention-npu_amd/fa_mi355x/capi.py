"""ctypes binding of the C ABI in include/fa_mi355x.h (libfa_mi355x.so).

This is the binding a host without PyTorch C++ would use (the reference binds
its host functions with pybind11 instead: csrc/arch22/flash_attn_npu_v2/
flash_api.cpp:1301-1309). The torch operators in libfa_mi355x_torch.so call the
same entry points; tests use this module to call the library directly.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
CORE_LIB = os.path.join(_HERE, "lib", "libfa_mi355x.so")

ABI_VERSION = 4
FA_OK, FA_EINVAL, FA_EUNSUPPORTED, FA_EHIP, FA_EWORKSPACE = 0, 1, 2, 3, 4
FA_DTYPE_FP16, FA_DTYPE_BF16, FA_DTYPE_FP32, FA_DTYPE_FP8_E4M3 = 0, 1, 2, 3
FA_KIND_KVCACHE, FA_KIND_DENSE, FA_KIND_VARLEN = 0, 1, 2

EXPORTED = ["fa_abi_version", "fa_validate", "fa_fwd_workspace_size", "fa_mha_fwd_kvcache", "fa_mha_fwd",
            "fa_mha_varlen_fwd", "fa_mha_fwd_kvcache_noalloc", "fa_combine", "fa_last_error", "fa_validate_bwd",
            "fa_bwd_workspace_size", "fa_mha_bwd", "fa_mha_varlen_bwd"]
NOALLOC_SCRATCH_BYTES = 32 << 20  # FA_NOALLOC_SCRATCH_BYTES

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


class FwdParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32), ("dtype", _i32),
        ("batch", _i32), ("seqlen_q", _i32), ("nheads", _i32), ("nheads_k", _i32),
        ("headdim", _i32), ("headdim_v", _i32), ("seqlen_k", _i32), ("batch_cache", _i32), ("total_q", _i32),
        ("q", _vp), ("q_batch_stride", _i64), ("q_row_stride", _i64), ("q_head_stride", _i64),
        ("k", _vp), ("k_batch_stride", _i64), ("k_row_stride", _i64), ("k_head_stride", _i64),
        ("v", _vp), ("v_batch_stride", _i64), ("v_row_stride", _i64), ("v_head_stride", _i64),
        ("k_new", _vp), ("knew_batch_stride", _i64), ("knew_row_stride", _i64), ("knew_head_stride", _i64),
        ("v_new", _vp), ("vnew_batch_stride", _i64), ("vnew_row_stride", _i64), ("vnew_head_stride", _i64),
        ("seqlen_new", _i32),
        ("out", _vp), ("out_batch_stride", _i64), ("out_row_stride", _i64), ("out_head_stride", _i64),
        ("softmax_lse", _vp),
        ("cache_seqlens", _vp), ("cu_seqlens_q", _vp), ("cu_seqlens_k", _vp),
        ("block_table", _vp), ("block_table_batch_stride", _i64), ("max_blocks_per_seq", _i32), ("block_table_rows", _i32),
        ("page_block_size", _i32), ("cache_batch_idx", _vp),
        ("rotary_cos", _vp), ("rotary_sin", _vp), ("rotary_dim", _i32), ("seqlen_ro", _i32),
        ("rotary_interleaved", _i32),
        ("alibi_slopes", _vp), ("alibi_batch_stride", _i64),
        ("softmax_scale", ctypes.c_float), ("softcap", ctypes.c_float), ("dropout_p", ctypes.c_float),
        ("is_causal", _i32), ("window_size_left", _i32), ("window_size_right", _i32), ("num_splits", _i32),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("stage_events", _vp),
        ("cache_leftpad", _vp), ("cu_seqlens_k_new", _vp), ("total_k_new", _i32), ("rotary_seqlens", _vp),
        ("attention_chunk", _i32),
        ("q_descale", _vp), ("q_descale_batch_stride", _i64), ("q_descale_head_stride", _i64),
        ("k_descale", _vp), ("k_descale_batch_stride", _i64), ("k_descale_head_stride", _i64),
        ("v_descale", _vp), ("v_descale_batch_stride", _i64), ("v_descale_head_stride", _i64),
        ("qv", _vp), ("qv_batch_stride", _i64), ("qv_row_stride", _i64), ("qv_head_stride", _i64),
        ("no_pack_gqa", _i32),
    ]


class BwdParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32), ("dtype", _i32),
        ("batch", _i32), ("seqlen_q", _i32), ("seqlen_k", _i32), ("nheads", _i32), ("nheads_k", _i32),
        ("headdim", _i32), ("total_q", _i32),
        ("q", _vp), ("q_batch_stride", _i64), ("q_row_stride", _i64), ("q_head_stride", _i64),
        ("k", _vp), ("k_batch_stride", _i64), ("k_row_stride", _i64), ("k_head_stride", _i64),
        ("v", _vp), ("v_batch_stride", _i64), ("v_row_stride", _i64), ("v_head_stride", _i64),
        ("out", _vp), ("out_batch_stride", _i64), ("out_row_stride", _i64), ("out_head_stride", _i64),
        ("dout", _vp), ("dout_batch_stride", _i64), ("dout_row_stride", _i64), ("dout_head_stride", _i64),
        ("dq", _vp), ("dq_batch_stride", _i64), ("dq_row_stride", _i64), ("dq_head_stride", _i64),
        ("dk", _vp), ("dk_batch_stride", _i64), ("dk_row_stride", _i64), ("dk_head_stride", _i64),
        ("dv", _vp), ("dv_batch_stride", _i64), ("dv_row_stride", _i64), ("dv_head_stride", _i64),
        ("softmax_lse", _vp), ("softmax_d", _vp),
        ("cu_seqlens_q", _vp), ("cu_seqlens_k", _vp),
        ("alibi_slopes", _vp), ("alibi_batch_stride", _i64),
        ("softmax_scale", ctypes.c_float), ("softcap", ctypes.c_float), ("dropout_p", ctypes.c_float),
        ("is_causal", _i32), ("window_size_left", _i32), ("window_size_right", _i32), ("deterministic", _i32),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("attention_chunk", _i32),
    ]


_lib = None


def lib():
    """Load libfa_mi355x.so (raises OSError when it is not built)."""
    global _lib
    if _lib is None:
        L = ctypes.CDLL(CORE_LIB)
        P = ctypes.POINTER(FwdParams)
        L.fa_abi_version.restype = ctypes.c_int
        L.fa_validate.argtypes = [P, _i32]
        L.fa_validate.restype = ctypes.c_int
        L.fa_fwd_workspace_size.argtypes = [P, _i32, ctypes.POINTER(ctypes.c_size_t)]
        L.fa_fwd_workspace_size.restype = ctypes.c_int
        for fn in ("fa_mha_fwd_kvcache", "fa_mha_fwd", "fa_mha_varlen_fwd", "fa_mha_fwd_kvcache_noalloc"):
            getattr(L, fn).argtypes = [P, _vp]
            getattr(L, fn).restype = ctypes.c_int
        L.fa_combine.argtypes = [_vp, _vp, _i32, _i64, _i32, _vp, _i64, _i32, _vp, _vp]
        L.fa_combine.restype = ctypes.c_int
        L.fa_last_error.restype = ctypes.c_char_p
        PB = ctypes.POINTER(BwdParams)
        L.fa_validate_bwd.argtypes = [PB, _i32]
        L.fa_validate_bwd.restype = ctypes.c_int
        L.fa_bwd_workspace_size.argtypes = [PB, _i32, ctypes.POINTER(ctypes.c_size_t)]
        L.fa_bwd_workspace_size.restype = ctypes.c_int
        for fn in ("fa_mha_bwd", "fa_mha_varlen_bwd"):
            getattr(L, fn).argtypes = [PB, _vp]
            getattr(L, fn).restype = ctypes.c_int
        _lib = L
    return _lib


def last_error():
    return lib().fa_last_error().decode()


def new_params(**kw):
    p = FwdParams()
    p.abi_version = ABI_VERSION
    p.window_size_left = -1
    p.window_size_right = -1
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def validate(p, kind):
    return lib().fa_validate(ctypes.byref(p), kind)


def workspace_size(p, kind):
    n = ctypes.c_size_t(0)
    st = lib().fa_fwd_workspace_size(ctypes.byref(p), kind, ctypes.byref(n))
    return st, n.value


_ENTRY = {FA_KIND_KVCACHE: "fa_mha_fwd_kvcache", FA_KIND_DENSE: "fa_mha_fwd", FA_KIND_VARLEN: "fa_mha_varlen_fwd"}


def forward(p, kind, stream=0):
    return getattr(lib(), _ENTRY[kind])(ctypes.byref(p), stream)


def forward_kvcache_noalloc(p, stream=0):
    """fa_mha_fwd_kvcache_noalloc: p.workspace is ignored (library scratch)."""
    return lib().fa_mha_fwd_kvcache_noalloc(ctypes.byref(p), stream)


def new_bwd_params(**kw):
    p = BwdParams()
    p.abi_version = ABI_VERSION
    p.window_size_left = -1
    p.window_size_right = -1
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def validate_bwd(p, kind):
    return lib().fa_validate_bwd(ctypes.byref(p), kind)


def backward(p, kind, stream=0):
    fn = lib().fa_mha_varlen_bwd if kind == FA_KIND_VARLEN else lib().fa_mha_bwd
    return fn(ctypes.byref(p), stream)
