"""Python front of the CPU checker (oracle/fa_oracle.c).

TEST INFRASTRUCTURE ONLY. tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module to check the HIP path; the product never
does. Arrays are numpy: 16-bit floats travel as raw uint16 bit patterns so the
append / rotary checks can be bit-exact.

`kvcache_forward` restates the whole `flash_attn_with_kvcache` contract
(flash_attn_npu_v2/interface_arch22.py:1452-1538 in the reference):
append (after rotary) at cache_seqlens, rotary on q, then the blockwise golden
`ref_flash_attention` (tests/test_flash_attn_npu_v3.py:87-146) over the
L_b + S_new keys of each sequence, with bottom-right causal / local masks
(tests/fa_small_op_golden.py:21-58).
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libfa_oracle.so")

FP16, BF16 = 0, 1

_i64 = ctypes.c_int64
_i32p = ctypes.POINTER(ctypes.c_int32)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_f32p = ctypes.POINTER(ctypes.c_float)


class _FwdParams(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int), ("B", ctypes.c_int), ("Sq", ctypes.c_int), ("Sk", ctypes.c_int),
        ("H", ctypes.c_int), ("Hk", ctypes.c_int), ("D", ctypes.c_int), ("Dv", ctypes.c_int),
        ("q", _u16p), ("q_sb", _i64), ("q_si", _i64), ("q_sh", _i64),
        ("cu_seqlens_q", _i32p),
        ("k", _u16p), ("k_sb", _i64), ("k_si", _i64), ("k_sh", _i64),
        ("v", _u16p), ("v_sb", _i64), ("v_si", _i64), ("v_sh", _i64),
        ("seqlens_k", _i32p), ("cu_seqlens_k", _i32p),
        ("block_table", _i32p), ("bt_stride", _i64), ("page", ctypes.c_int),
        ("batch_idx", _i32p),
        ("alibi", _f32p), ("alibi_sb", _i64),
        ("scale", ctypes.c_float), ("softcap", ctypes.c_float),
        ("wl", ctypes.c_int), ("wr", ctypes.c_int),
        ("out", _u16p), ("o_sb", _i64), ("o_si", _i64), ("o_sh", _i64),
        ("lse", _f32p), ("lse_sb", _i64), ("lse_sh", _i64),
        ("nthreads", ctypes.c_int),
        ("chunk", ctypes.c_int),
        ("qv", _u16p), ("qv_sb", _i64), ("qv_si", _i64), ("qv_sh", _i64),
    ]


class _RotaryParams(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int), ("B", ctypes.c_int), ("S", ctypes.c_int), ("H", ctypes.c_int),
        ("D", ctypes.c_int), ("rotary_dim", ctypes.c_int), ("interleaved", ctypes.c_int),
        ("q_same_pos", ctypes.c_int),
        ("x", _u16p), ("x_sb", _i64), ("x_si", _i64), ("x_sh", _i64),
        ("seqlens", _i32p), ("cos", _u16p), ("sin", _u16p), ("cs_stride", _i64),
    ]


class _AppendParams(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int), ("B", ctypes.c_int), ("S_new", ctypes.c_int), ("Hk", ctypes.c_int),
        ("D", ctypes.c_int), ("Dv", ctypes.c_int), ("rotary_dim", ctypes.c_int),
        ("interleaved", ctypes.c_int),
        ("k_new", _u16p), ("v_new", _u16p), ("n_sb", _i64), ("n_si", _i64), ("n_sh", _i64),
        ("k_cache", _u16p), ("v_cache", _u16p), ("c_sb", _i64), ("c_si", _i64), ("c_sh", _i64),
        ("seqlens", _i32p), ("batch_idx", _i32p),
        ("block_table", _i32p), ("bt_stride", _i64), ("page", ctypes.c_int),
        ("cos", _u16p), ("sin", _u16p), ("cs_stride", _i64),
        ("rot_pos", _i32p),
    ]


_lib = None


def build():
    """Compile the checker with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_attention.argtypes = [ctypes.POINTER(_FwdParams)]
        L.orc_rotary_q.argtypes = [ctypes.POINTER(_RotaryParams)]
        L.orc_kv_append.argtypes = [ctypes.POINTER(_AppendParams)]
        L.orc_combine.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int, _f32p, _f32p, _f32p, _f32p]
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_bf16_to_f32.restype = ctypes.c_float
        L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _p(a, t):
    if a is None:
        return ctypes.cast(None, ctypes.POINTER(t))
    assert a.flags["C_CONTIGUOUS"] or a.ndim == 0
    return a.ctypes.data_as(ctypes.POINTER(t))


def _st(a):
    """Element strides of a numpy array."""
    return [s // a.itemsize for s in a.strides]


# ---- dtype helpers ---------------------------------------------------------------

def to_bits(x, dtype):
    """float array -> uint16 bit patterns, RNE (bf16) / IEEE (fp16)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == FP16:
        return x.astype(np.float16).view(np.uint16)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def from_bits(b, dtype):
    b = np.ascontiguousarray(b, dtype=np.uint16)
    if dtype == FP16:
        return b.view(np.float16).astype(np.float32)
    return (b.astype(np.uint32) << 16).view(np.float32)


def normalize_window(seqlen_q, seqlen_k, causal, wl, wr):
    """tests/fa_small_op_golden.py:21-32."""
    if wl >= seqlen_k - 1:
        wl = -1
    if wr >= seqlen_q - 1:
        wr = -1
    if causal:
        wr = 0
    return wl, wr


# ---- attention ---------------------------------------------------------------------

def attention(q, k, v, *, dtype, scale, softcap=0.0, causal=False, window=(-1, -1), alibi=None,
              seqlens_k=None, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=None,
              block_table=None, batch_idx=None, nthreads=1, chunk=0, qv=None):
    """Blockwise golden forward.

    q: (B, Sq, H, D) or, with cu_seqlens_q, (T, H, D) uint16 bits.
    qv: None, or rows like q with v's head dim; the scores add qv . v.
    k, v: (Bc, Sk, Hk, D) contiguous caches, (num_blocks, page, Hk, D) with block_table,
          or (Tk, Hk, D) with cu_seqlens_k.
    Returns (out uint16 like q, lse float32 (B, H, Sq) or (H, T)).
    """
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    varlen_q = cu_seqlens_q is not None
    if varlen_q:
        T, H, D = q.shape
        cu_q = np.ascontiguousarray(cu_seqlens_q, dtype=np.int32)
        B = len(cu_q) - 1
        Sq = int(max_seqlen_q if max_seqlen_q is not None else np.max(np.diff(cu_q)) if B else 0)
        q_st = [0] + _st(q)
    else:
        B, Sq, H, D = q.shape
        cu_q = None
        q_st = _st(q)
    if cu_seqlens_k is not None:
        Hk, Dv = k.shape[-2], v.shape[-1]
        k_st = [0] + _st(k)
        v_st = [0] + _st(v)
        Sk = 0
    else:
        Hk, Dv = k.shape[2], v.shape[3]
        k_st, v_st = _st(k), _st(v)
        Sk = k.shape[1] if block_table is None else block_table.shape[1] * k.shape[1]
    # The window is normalised per call (seqlens-independent rules are a
    # no-op on the mask itself, only the causal flag forces wr = 0).
    wl, wr = window
    if causal:
        wr = 0
    out = np.zeros(q.shape[:-1] + (Dv,), dtype=np.uint16)
    if varlen_q:
        lse = np.full((H, q.shape[0]), np.inf, dtype=np.float32)
        o_st = [0] + _st(out)
        lse_sb, lse_sh = 0, lse.shape[1]
    else:
        lse = np.full((B, H, Sq), np.inf, dtype=np.float32)
        o_st = _st(out)
        lse_sb, lse_sh = H * Sq, Sq
    keep = []

    def i32(a):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dtype=np.int32)
        keep.append(a)
        return a
    seqlens_k = i32(seqlens_k)
    cu_k = i32(cu_seqlens_k)
    bt = i32(block_table)
    bidx = i32(batch_idx)
    al = None
    al_sb = 0
    if alibi is not None:
        al = np.ascontiguousarray(alibi, dtype=np.float32)
        al_sb = H if al.ndim == 2 else 0
    p = _FwdParams(
        dtype=dtype, B=B, Sq=Sq, Sk=Sk, H=H, Hk=Hk, D=D, Dv=Dv,
        q=_p(q, ctypes.c_uint16), q_sb=q_st[0], q_si=q_st[1], q_sh=q_st[2],
        cu_seqlens_q=_p(cu_q, ctypes.c_int32),
        k=_p(k, ctypes.c_uint16), k_sb=k_st[0], k_si=k_st[1], k_sh=k_st[2],
        v=_p(v, ctypes.c_uint16), v_sb=v_st[0], v_si=v_st[1], v_sh=v_st[2],
        seqlens_k=_p(seqlens_k, ctypes.c_int32), cu_seqlens_k=_p(cu_k, ctypes.c_int32),
        block_table=_p(bt, ctypes.c_int32), bt_stride=(bt.shape[1] if bt is not None else 0),
        page=(k.shape[1] if bt is not None else 0),
        batch_idx=_p(bidx, ctypes.c_int32),
        alibi=_p(al, ctypes.c_float), alibi_sb=al_sb,
        scale=scale, softcap=softcap, wl=wl, wr=wr,
        out=_p(out, ctypes.c_uint16), o_sb=o_st[0], o_si=o_st[1], o_sh=o_st[2],
        lse=_p(lse, ctypes.c_float), lse_sb=lse_sb, lse_sh=lse_sh,
        nthreads=nthreads, chunk=int(chunk),
    )
    if qv is not None:
        qv = np.ascontiguousarray(qv)
        assert qv.shape[:-1] == q.shape[:-1] and qv.shape[-1] == Dv, "qv must be q's rows with v's head dim"
        qst = ([0] + _st(qv)) if varlen_q else _st(qv)
        p.qv = _p(qv, ctypes.c_uint16)
        p.qv_sb, p.qv_si, p.qv_sh = qst[0], qst[1], qst[2]
    rc = lib().orc_attention(ctypes.byref(p))
    if rc != 0:
        raise ValueError("oracle rejected the shapes")
    return out, lse


def e4m3_to_bf16_bits(x8):
    """OCP 8-bit floating point E4M3 ("e4m3fn": torch.float8_e4m3fn) bytes ->
    bf16 bit patterns. Definition (OCP 8-bit Floating Point Specification
    v1.0, E4M3): sign bit, 4-bit exponent with bias 7, 3-bit mantissa;
    exponent 0 is subnormal (m/8 * 2^-6); S.1111.111 is NaN; no infinities.
    Every E4M3 value has at most 4 significant bits, so the bf16 pattern is
    the exact value. Used for the FP8 inputs of the v3 API (q_descale /
    k_descale / v_descale, flash_attn_npu_v3/interface_arch22.py:797-965 of
    the reference, which rejects them at csrc/arch22/flash_attn_npu_v3/
    flash_api.cpp:154-156)."""
    x = np.asarray(x8, dtype=np.uint8).astype(np.int32)
    s = (x >> 7) & 1
    e = (x >> 3) & 15
    m = x & 7
    val = np.where(e > 0, np.ldexp(1.0 + m / 8.0, e - 7), np.ldexp(m / 8.0, -6))
    val = np.where(s == 1, -val, val).astype(np.float32)
    val = np.where((e == 15) & (m == 7), np.float32(np.nan), val)
    return (val.view(np.uint32) >> 16).astype(np.uint16)


def attention_fp8(q8, k8, v8, *, scale, q_descale=None, k_descale=None, v_descale=None, causal=False,
                  window=(-1, -1), softcap=0.0, seqlens_k=None, nthreads=1):
    """FP8 forward on (B, S, H, D) q and (B, Sk, Hk, D) k / v e4m3 bytes
    (dense, or a contiguous cache with seqlens_k): the values widen exactly
    to bf16 and, for sequence b and kv head hk, the scores use
    scale * q_descale[b, hk] * k_descale[b, hk] and the output is multiplied
    by v_descale[b, hk] (descales (B, Hk) fp32, None = 1). Runs the blockwise
    golden per (b, hk) with that scale and bf16 arithmetic.
    Returns (out float32 like q, lse float32 (B, H, Sq))."""
    q = e4m3_to_bf16_bits(q8)
    k = e4m3_to_bf16_bits(k8)
    v = e4m3_to_bf16_bits(v8)
    B, Sq, H, D = q.shape
    Hk = k.shape[2]
    g = H // Hk
    one = np.ones((B, Hk), dtype=np.float32)
    qd = one if q_descale is None else np.asarray(q_descale, dtype=np.float32)
    kd = one if k_descale is None else np.asarray(k_descale, dtype=np.float32)
    vd = one if v_descale is None else np.asarray(v_descale, dtype=np.float32)
    out = np.zeros((B, Sq, H, v.shape[3]), dtype=np.float32)
    lse = np.zeros((B, H, Sq), dtype=np.float32)
    for b in range(B):
        for hk in range(Hk):
            sc = float(np.float32(scale) * qd[b, hk] * kd[b, hk])
            o, l = attention(q[b:b + 1, :, hk * g:(hk + 1) * g], k[b:b + 1, :, hk:hk + 1], v[b:b + 1, :, hk:hk + 1],
                             dtype=BF16, scale=sc, softcap=softcap, causal=causal, window=window,
                             seqlens_k=None if seqlens_k is None else np.asarray(seqlens_k)[b:b + 1],
                             nthreads=nthreads)
            out[b, :, hk * g:(hk + 1) * g] = from_bits(o, BF16)[0] * vd[b, hk]
            lse[b, hk * g:(hk + 1) * g] = l[0]
    return out, lse


def rotary(x, cos, sin, seqlens, *, dtype, interleaved, same_pos=False):
    """Rotary on (B, S, H, D) bits at positions seqlens[b] + i (or seqlens[b])."""
    x = np.array(x, dtype=np.uint16, copy=True, order="C")
    cos = np.ascontiguousarray(cos, dtype=np.uint16)
    sin = np.ascontiguousarray(sin, dtype=np.uint16)
    sl = np.ascontiguousarray(seqlens, dtype=np.int32)
    B, S, H, D = x.shape
    st = _st(x)
    p = _RotaryParams(dtype=dtype, B=B, S=S, H=H, D=D, rotary_dim=2 * cos.shape[1],
                      interleaved=int(interleaved), q_same_pos=int(same_pos),
                      x=_p(x, ctypes.c_uint16), x_sb=st[0], x_si=st[1], x_sh=st[2],
                      seqlens=_p(sl, ctypes.c_int32), cos=_p(cos, ctypes.c_uint16),
                      sin=_p(sin, ctypes.c_uint16), cs_stride=cos.shape[1])
    lib().orc_rotary_q(ctypes.byref(p))
    return x


def kv_append(k_cache, v_cache, k_new, v_new, seqlens, *, dtype, batch_idx=None, block_table=None,
              cos=None, sin=None, interleaved=True, rot_pos=None):
    """In-place append (after rotary on k) into copies of the caches; returns them.
    Token t of batch b goes to slot seqlens[b] + t and is rotated at rot_pos[b] + t
    (default: at its slot)."""
    kc = np.array(k_cache, dtype=np.uint16, copy=True, order="C")
    vc = np.array(v_cache, dtype=np.uint16, copy=True, order="C")
    kn = np.ascontiguousarray(k_new, dtype=np.uint16)
    vn = np.ascontiguousarray(v_new, dtype=np.uint16)
    sl = np.ascontiguousarray(seqlens, dtype=np.int32)
    bidx = None if batch_idx is None else np.ascontiguousarray(batch_idx, dtype=np.int32)
    bt = None if block_table is None else np.ascontiguousarray(block_table, dtype=np.int32)
    if cos is not None:
        cos = np.ascontiguousarray(cos, dtype=np.uint16)
        sin = np.ascontiguousarray(sin, dtype=np.uint16)
    rp = None if rot_pos is None else np.ascontiguousarray(rot_pos, dtype=np.int32)
    B, S_new, Hk, D = kn.shape
    nst = _st(kn)
    cst = _st(kc)
    p = _AppendParams(dtype=dtype, B=B, S_new=S_new, Hk=Hk, D=D, Dv=vn.shape[3],
                      rotary_dim=(2 * cos.shape[1] if cos is not None else 0),
                      interleaved=int(interleaved),
                      k_new=_p(kn, ctypes.c_uint16), v_new=_p(vn, ctypes.c_uint16),
                      n_sb=nst[0], n_si=nst[1], n_sh=nst[2],
                      k_cache=_p(kc, ctypes.c_uint16), v_cache=_p(vc, ctypes.c_uint16),
                      c_sb=cst[0], c_si=cst[1], c_sh=cst[2],
                      seqlens=_p(sl, ctypes.c_int32), batch_idx=_p(bidx, ctypes.c_int32),
                      block_table=_p(bt, ctypes.c_int32),
                      bt_stride=(bt.shape[1] if bt is not None else 0),
                      page=(kc.shape[1] if bt is not None else 0),
                      cos=_p(cos, ctypes.c_uint16), sin=_p(sin, ctypes.c_uint16),
                      cs_stride=(cos.shape[1] if cos is not None else 0),
                      rot_pos=_p(rp, ctypes.c_int32))
    lib().orc_kv_append(ctypes.byref(p))
    return kc, vc


def combine(o_part, lse_part):
    """o_part (S, R, Dv) fp32, lse_part (S, R) -> (o (R, Dv), lse (R,))."""
    o_part = np.ascontiguousarray(o_part, dtype=np.float32)
    lse_part = np.ascontiguousarray(lse_part, dtype=np.float32)
    S, R, Dv = o_part.shape
    o = np.zeros((R, Dv), dtype=np.float32)
    lse = np.zeros((R,), dtype=np.float32)
    lib().orc_combine(S, R, Dv, _p(o_part, ctypes.c_float), _p(lse_part, ctypes.c_float),
                      _p(o, ctypes.c_float), _p(lse, ctypes.c_float))
    return o, lse


def kvcache_forward(q, k_cache, v_cache, *, dtype, cache_seqlens, k=None, v=None, rotary_cos=None,
                    rotary_sin=None, rotary_interleaved=True, cache_batch_idx=None, block_table=None,
                    softmax_scale=None, causal=False, window=(-1, -1), softcap=0.0, alibi=None,
                    nthreads=1):
    """The flash_attn_with_kvcache contract on host arrays.

    Returns (out, lse, k_cache_after, v_cache_after)."""
    B, Sq, H, D = q.shape
    seqlens = np.ascontiguousarray(cache_seqlens, dtype=np.int32)
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    kc, vc = k_cache, v_cache
    s_new = 0
    if k is not None:
        s_new = k.shape[1]
        kc, vc = kv_append(k_cache, v_cache, k, v, seqlens, dtype=dtype, batch_idx=cache_batch_idx,
                           block_table=block_table, cos=rotary_cos, sin=rotary_sin,
                           interleaved=rotary_interleaved)
        if rotary_cos is not None:
            same = not (causal or window[0] >= 0 or window[1] >= 0)
            q = rotary(q, rotary_cos, rotary_sin, seqlens, dtype=dtype, interleaved=rotary_interleaved,
                       same_pos=same)
    out, lse = attention(q, kc, vc, dtype=dtype, scale=softmax_scale, softcap=softcap, causal=causal,
                         window=window, alibi=alibi, seqlens_k=seqlens + s_new,
                         block_table=block_table, batch_idx=cache_batch_idx, nthreads=nthreads)
    return out, lse, kc, vc


def kvcache_forward_v3(q, k_cache, v_cache, *, dtype, cache_seqlens, k=None, v=None, rotary_cos=None,
                       rotary_sin=None, rotary_interleaved=True, cache_batch_idx=None, block_table=None,
                       softmax_scale=None, causal=False, window=(-1, -1), softcap=0.0, alibi=None,
                       cache_leftpad=None, rotary_seqlens=None, cu_seqlens_q=None, max_seqlen_q=None,
                       cu_seqlens_k_new=None, attention_chunk=0, nthreads=1, qv=None):
    """The v3 flash_attn_with_kvcache contract (README.md:311-401 of the
    reference, whose kernels reject the extensions), one sequence at a time:

      * q is (B, Sq, H, D), or (total_q, H, D) split by cu_seqlens_q;
      * k / v are (B, S_new, Hk, D), or (total_k_new, Hk, D) split by
        cu_seqlens_k_new; token t of sequence b is appended at slot
        L_b + t (L = cache_seqlens) and rotated at P_b + t, where
        P = rotary_seqlens (default L);
      * q row i of sequence b is rotated at P_b + i (causal or local) or P_b;
      * the keys of sequence b are cache slots [lp_b, L_b + S_new(b)) with
        lp = cache_leftpad (default 0): attention runs on the cache with its
        first lp_b slots removed, so masks count keys from lp_b;
      * attention_chunk c > 0 also restricts query i to the chunk of its
        diagonal key;
      * qv (rows like q, v's head dim) adds qv . v to the scores, and the
        default scale is then (D + Dv) ** -0.5 (FlashAttention-3).

    Built from the pinned primitives kv_append, rotary and attention.
    Returns (out, lse, k_cache_after, v_cache_after); lse is (B, H, Sq), or
    (H, total_q) for ragged q."""
    ragged_q = cu_seqlens_q is not None
    cu_q = None if not ragged_q else np.asarray(cu_seqlens_q, dtype=np.int64)
    B = len(cu_q) - 1 if ragged_q else q.shape[0]
    H, D = q.shape[-2], q.shape[-1]
    if softmax_scale is None:
        softmax_scale = (D + (qv.shape[-1] if qv is not None else 0)) ** -0.5
    L = np.asarray(cache_seqlens, dtype=np.int64)
    P = L if rotary_seqlens is None else np.asarray(rotary_seqlens, dtype=np.int64)
    lp = np.zeros(B, np.int64) if cache_leftpad is None else np.asarray(cache_leftpad, dtype=np.int64)
    crow = np.arange(B) if cache_batch_idx is None else np.asarray(cache_batch_idx, dtype=np.int64)
    cu_n = None if cu_seqlens_k_new is None else np.asarray(cu_seqlens_k_new, dtype=np.int64)
    kc = np.array(k_cache, dtype=np.uint16, copy=True, order="C")
    vc = np.array(v_cache, dtype=np.uint16, copy=True, order="C")
    out = np.zeros(q.shape, dtype=np.uint16)
    if ragged_q:
        lse = np.full((H, q.shape[0]), np.inf, dtype=np.float32)
    else:
        lse = np.full((B, H, q.shape[1]), np.inf, dtype=np.float32)
    same = not (causal or window[0] >= 0 or window[1] >= 0)
    for b in range(B):
        s_new = 0
        if k is not None:
            if cu_n is not None:
                kb, vb = k[cu_n[b]:cu_n[b + 1]][None], v[cu_n[b]:cu_n[b + 1]][None]
            else:
                kb, vb = k[b:b + 1], v[b:b + 1]
            s_new = kb.shape[1]
            if s_new > 0:
                kc, vc = kv_append(kc, vc, kb, vb, L[b:b + 1], dtype=dtype, batch_idx=crow[b:b + 1],
                                   block_table=block_table, cos=rotary_cos, sin=rotary_sin,
                                   interleaved=rotary_interleaved, rot_pos=P[b:b + 1])
        qb = q[cu_q[b]:cu_q[b + 1]][None] if ragged_q else q[b:b + 1]
        qvb = None if qv is None else (qv[cu_q[b]:cu_q[b + 1]][None] if ragged_q else qv[b:b + 1])
        if qb.shape[1] == 0:
            continue
        if k is not None and rotary_cos is not None:
            qb = rotary(qb, rotary_cos, rotary_sin, P[b:b + 1], dtype=dtype, interleaved=rotary_interleaved,
                        same_pos=same)
        if block_table is None:
            kv_k, kv_v = kc[crow[b]:crow[b] + 1, lp[b]:], vc[crow[b]:crow[b] + 1, lp[b]:]
            bidx = None
        else:
            kv_k, kv_v, bidx = kc, vc, crow[b:b + 1]
        ab = None
        if alibi is not None:
            al = np.asarray(alibi, dtype=np.float32)
            ab = al[b] if al.ndim == 2 else al
        ob, lb = attention(qb, kv_k, kv_v, dtype=dtype, scale=softmax_scale, softcap=softcap, causal=causal,
                           window=window, alibi=ab, seqlens_k=np.array([L[b] + s_new - lp[b]]),
                           block_table=block_table, batch_idx=bidx, nthreads=nthreads, chunk=attention_chunk,
                           qv=qvb)
        if ragged_q:
            out[cu_q[b]:cu_q[b + 1]] = ob[0]
            lse[:, cu_q[b]:cu_q[b + 1]] = lb[0]
        else:
            out[b] = ob[0]
            lse[b] = lb[0]
    return out, lse, kc, vc
