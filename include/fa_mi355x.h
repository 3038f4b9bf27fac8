/*
 * fa_mi355x.h -- C ABI of the MI355X (gfx950) FlashAttention library
 * (libfa_mi355x.so). Plain pointers, sizes and a stream handle: no torch or
 * HIP types, so any FFI (ctypes, cgo, JNI, N-API) can bind it.
 *
 * The entry points replace the reference's pybind11 functions
 * (paths relative to the reference repository):
 *   fa_mha_fwd_kvcache  <- mha_fwd_kvcache  csrc/arch22/flash_attn_npu_v2/flash_api.cpp:356-626
 *                          (bound as fwd_kvcache at flash_api.cpp:1306) and the kvcache branch of
 *                          mha_fwd           csrc/arch22/flash_attn_npu_v3/flash_api.cpp:60-491
 *   fa_mha_fwd          <- mha_fwd          csrc/arch22/flash_attn_npu_v2/flash_api.cpp:628-826
 *                          (bound as fwd at flash_api.cpp:1303)
 *   fa_mha_varlen_fwd   <- mha_varlen_fwd   csrc/arch22/flash_attn_npu_v2/flash_api.cpp:828-1060
 *                          (bound as varlen_fwd at flash_api.cpp:1304)
 *   fa_fwd_workspace_size / fa_validate
 *                       <- the host-side validation and workspace sizing inside those
 *                          functions (flash_api.cpp:382-441 and :541-565)
 *   fa_combine          <- CombineScale (csrc/arch22/flash_attn_npu_v2/CombineScale.hpp:76-357),
 *                          exposed as the v3 flash_attn_combine
 *                          (flash_attn_npu_v3/interface_arch22.py:930-931)
 *   fa_mha_bwd          <- mha_bwd          csrc/arch22/flash_attn_npu_v2/flash_api.cpp:1251-1299
 *                          (bound as bwd at flash_api.cpp:1305)
 *   fa_mha_varlen_bwd   <- mha_varlen_bwd   csrc/arch22/flash_attn_npu_v2/flash_api.cpp:1063-1249
 *                          (bound as varlen_bwd)
 *   fa_validate_bwd     <- the host-side checks of those two functions
 *
 * Conventions
 *   - All tensor strides are in ELEMENTS; the last (head) dimension must be
 *     contiguous and every row start 16-byte aligned.
 *   - The library never allocates or frees device memory. The caller passes a
 *     workspace of at least fa_fwd_workspace_size() bytes (256-byte aligned).
 *   - Every function returns FA_OK or an error code; fa_last_error() gives a
 *     thread-local message for the last failure on the calling thread.
 *   - Work is enqueued on `stream` (a hipStream_t, or NULL for the null
 *     stream). Nothing synchronises the host and nothing reads device memory
 *     on the host.
 */
#ifndef FA_MI355X_H
#define FA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_MI355X_ABI_VERSION 4

typedef enum {
    FA_OK = 0,
    FA_EINVAL = 1,        /* invalid argument (shape, stride, value) */
    FA_EUNSUPPORTED = 2,  /* valid but not implemented (e.g. dropout) */
    FA_EHIP = 3,          /* HIP runtime error at launch */
    FA_EWORKSPACE = 4     /* workspace missing or too small */
} fa_status_t;

typedef enum {
    FA_DTYPE_FP16 = 0,
    FA_DTYPE_BF16 = 1,
    FA_DTYPE_FP32 = 2,     /* fa_combine output only */
    FA_DTYPE_FP8_E4M3 = 3  /* forward only: q, k, v, k_new, v_new in OCP float8 e4m3fn (torch.float8_e4m3fn),
                              out in bf16; see q_descale below */
} fa_dtype_t;

typedef enum {
    FA_KIND_KVCACHE = 0,  /* flash_attn_with_kvcache */
    FA_KIND_DENSE = 1,    /* flash_attn_func */
    FA_KIND_VARLEN = 2    /* flash_attn_varlen_func */
} fa_kind_t;

typedef struct fa_fwd_params {
    int32_t abi_version;  /* FA_MI355X_ABI_VERSION */
    int32_t dtype;        /* fa_dtype_t, shared by q, k, v, k_new, v_new, out, rotary cos/sin
                             (FP8_E4M3: out is bf16, no rotary) */

    int32_t batch;        /* B (query batch) */
    int32_t seqlen_q;     /* Sq (dense/kvcache), max_seqlen_q (varlen) */
    int32_t nheads;       /* H */
    int32_t nheads_k;     /* Hk, H % Hk == 0 */
    int32_t headdim;      /* D: a multiple of 8, at most 256 */
    int32_t headdim_v;    /* Dv (must equal D) */
    int32_t seqlen_k;     /* dense: Sk; kvcache contiguous: seqlen_cache; varlen: max_seqlen_k */
    int32_t batch_cache;  /* kvcache contiguous: rows of k/v cache; paged: num_blocks */
    int32_t total_q;      /* varlen: rows of q */

    /* q: (B, Sq, H, D) or varlen (total_q, H, D) */
    const void* q;
    int64_t q_batch_stride, q_row_stride, q_head_stride;
    /* k/v: dense (B, Sk, Hk, D); kvcache (Bc, Sc, Hk, D) or paged (num_blocks, page, Hk, D);
       varlen (total_k, Hk, D). Mutated in place when k_new/v_new are given. */
    void* k;
    int64_t k_batch_stride, k_row_stride, k_head_stride;
    void* v;
    int64_t v_batch_stride, v_row_stride, v_head_stride;
    /* kvcache only: new tokens (B, seqlen_new, Hk, D) appended at cache_seqlens */
    const void* k_new;
    int64_t knew_batch_stride, knew_row_stride, knew_head_stride;
    const void* v_new;
    int64_t vnew_batch_stride, vnew_row_stride, vnew_head_stride;
    int32_t seqlen_new;

    /* out: like q; softmax_lse: (B, H, Sq) fp32, varlen (H, total_q) fp32 */
    void* out;
    int64_t out_batch_stride, out_row_stride, out_head_stride;
    float* softmax_lse;

    const int32_t* cache_seqlens;   /* kvcache: (B,) int32, tokens already cached */
    const int32_t* cu_seqlens_q;    /* varlen: (B+1,) */
    const int32_t* cu_seqlens_k;    /* varlen: (B+1,) */
    const int32_t* block_table;     /* paged: (B or Bc, max_blocks) int32 */
    int64_t block_table_batch_stride;
    int32_t max_blocks_per_seq;
    int32_t block_table_rows;       /* rows of block_table (cache_batch_idx values index them) */
    int32_t page_block_size;
    const int32_t* cache_batch_idx; /* kvcache: (B,) rows of the cache / block table */

    const void* rotary_cos;         /* (seqlen_ro, rotary_dim/2), dtype as q */
    const void* rotary_sin;
    int32_t rotary_dim;
    int32_t seqlen_ro;
    int32_t rotary_interleaved;

    const float* alibi_slopes;      /* (H,) or (B, H) fp32 */
    int64_t alibi_batch_stride;     /* 0 for (H,), H for (B, H) */

    float softmax_scale;
    float softcap;                  /* 0 = off */
    float dropout_p;                /* must be 0 (forward inference only) */
    int32_t is_causal;
    int32_t window_size_left;       /* -1 = unbounded */
    int32_t window_size_right;
    int32_t num_splits;             /* 0 = heuristic, 1 = no split, n > 1 = n chunks */

    void* workspace;
    size_t workspace_bytes;

    /* Optional profiling hook: NULL, or 4 hipEvent_t handles recorded on
       `stream` before the KV append, before the attention kernel, before the
       split-KV combine and after the last kernel of the call. */
    void* const* stage_events;

    /* ---- kvcache extensions of the v3 API (all optional: NULL / 0 = off) ----
       The reference rejects these arguments (csrc/arch22/flash_attn_npu_v3/
       flash_api.cpp:150-162, v2 flash_api.cpp:416); the semantics are the
       flash_attn_with_kvcache docstring's (README.md:311-401 of the reference).
       The kvcache forward also takes cu_seqlens_q / total_q (above): q and out
       are then (total_q, H, D) and softmax_lse is (H, total_q). */
    const int32_t* cache_leftpad;    /* (B,): first valid row of each sequence's cache (contiguous caches);
                                        keys are cache rows [leftpad, cache_seqlens + new) */
    const int32_t* cu_seqlens_k_new; /* (B+1,): k_new / v_new are (total_k_new, Hk, D) and sequence b
                                        appends cu[b+1] - cu[b] tokens */
    int32_t total_k_new;             /* rows of k_new / v_new with cu_seqlens_k_new */
    const int32_t* rotary_seqlens;   /* (B,): rotary position of the first new token / query
                                        (default cache_seqlens) */
    int32_t attention_chunk;         /* > 0: a query sees only keys of its own chunk
                                        [c*floor(p/c), c*floor(p/c) + c) of its diagonal position p,
                                        intersected with the causal / local window */

    /* ---- FP8 inputs (dtype FA_DTYPE_FP8_E4M3; ABI 3) ----
       Descale factors of the v3 API (q_descale / k_descale / v_descale of
       flash_attn_func, flash_attn_varlen_func and flash_attn_with_kvcache,
       flash_attn_npu_v3/interface_arch22.py:797-965; the reference declares them
       (b, h_k) at csrc/arch22/flash_attn_npu_v3/flash_api.cpp:82-84 and rejects
       them at :154-156): fp32, shape (B, Hk),
       strides in elements; NULL = 1. With x8 the stored e4m3 values, sequence b
       and kv head hk = h / (H / Hk):
         scores = softmax_scale * q_descale[b,hk] * k_descale[b,hk] * (q8 . k8)
         out    = v_descale[b,hk] * softmax(scores) . v8
       The softmax_lse is that of these scores. headdim must be a multiple of
       16; rotary and the backward are not available for FP8. */
    const float* q_descale;
    int64_t q_descale_batch_stride, q_descale_head_stride;
    const float* k_descale;
    int64_t k_descale_batch_stride, k_descale_head_stride;
    const float* v_descale;
    int64_t v_descale_batch_stride, v_descale_head_stride;

    /* ---- qv and pack_gqa of the v3 API (ABI 4) ----
       flash_attn_npu_v3/interface_arch22.py:940-962 declares both; the
       reference kernels ignore qv (csrc/arch22/flash_attn_npu_v3/flash_api.cpp:66
       takes q_v_ and never reads it) and reject pack_gqa = True (:162). The
       semantics here are FlashAttention-3's:
         scores = softmax_scale * (q . k + qv . v)
       qv is (B, Sq, H, Dv), or (total_q, H, Dv) with cu_seqlens_q, in the
       dtype of q (16-bit only). It is taken by the decode kernel: at most 16
       query rows per kv head (seqlen_q * H / Hk, or seqlen_q with
       no_pack_gqa) and headdim <= 128; other shapes return FA_EUNSUPPORTED. */
    const void* qv;
    int64_t qv_batch_stride, qv_row_stride, qv_head_stride;
    /* nonzero (pack_gqa = False): each query head gets its own row tiles
       instead of sharing them with the other query heads of its kv head
       (GQA packing, the default). The results agree to rounding, not bit
       for bit: a wave rescales its rows' running maxima together when any
       of them needs it, so a row's rounding depends on the rows that share
       its wave, and the split-KV cuts may differ. The kv heads are then
       read once per query head instead of once. */
    int32_t no_pack_gqa;
} fa_fwd_params;

/* Library / ABI version. */
int fa_abi_version(void);

/* Host-only validation of `p` for the given kind; never touches the GPU. */
fa_status_t fa_validate(const fa_fwd_params* p, int32_t kind);

/* Bytes of workspace the call needs (host-only; 0 is possible). */
fa_status_t fa_fwd_workspace_size(const fa_fwd_params* p, int32_t kind, size_t* bytes);

/* Forward passes; enqueue on `stream` (hipStream_t). */
fa_status_t fa_mha_fwd_kvcache(const fa_fwd_params* p, void* stream);
fa_status_t fa_mha_fwd(const fa_fwd_params* p, void* stream);
fa_status_t fa_mha_varlen_fwd(const fa_fwd_params* p, void* stream);

/* No-allocation variant of fa_mha_fwd_kvcache. It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). p->workspace is ignored; the kernels' scratch is a device array
 * of FA_NOALLOC_SCRATCH_BYTES inside the library, one per GPU, held until the
 * process ends. A call whose fa_fwd_workspace_size exceeds that limit fails
 * with FA_EWORKSPACE. Calls that overlap on one GPU share the array and race:
 * serialise them. Nothing is allocated or freed. */
#define FA_NOALLOC_SCRATCH_BYTES (32u << 20)
fa_status_t fa_mha_fwd_kvcache_noalloc(const fa_fwd_params* p, void* stream);

/* Split-KV merge: out_partial (S, R, Dv) fp32, lse_partial (S, R) fp32 ->
 * out (R, Dv) in `out_dtype` (row stride out_row_stride elements),
 * lse (R,) fp32. Rows with no finite partial LSE get out = 0, lse = +inf. */
fa_status_t fa_combine(const float* out_partial, const float* lse_partial, int32_t num_splits, int64_t rows,
                       int32_t headdim_v, void* out, int64_t out_row_stride, int32_t out_dtype, float* lse,
                       void* stream);

/* ---- backward (dense / varlen) ------------------------------------------- */
typedef struct fa_bwd_params {
    int32_t abi_version;  /* FA_MI355X_ABI_VERSION */
    int32_t dtype;        /* fa_dtype_t of q, k, v, out, dout, dq, dk, dv */

    int32_t batch;        /* B */
    int32_t seqlen_q;     /* Sq (dense), max_seqlen_q (varlen) */
    int32_t seqlen_k;     /* Sk (dense), max_seqlen_k (varlen) */
    int32_t nheads;       /* H */
    int32_t nheads_k;     /* Hk, H % Hk == 0 */
    int32_t headdim;      /* D: a multiple of 8, at most 256 */
    int32_t total_q;      /* varlen: rows of q */

    /* q, out, dout, dq: (B, Sq, H, D) or varlen (total_q, H, D);
       k, v, dk, dv: (B, Sk, Hk, D) or varlen (total_k, Hk, D) */
    const void* q;
    int64_t q_batch_stride, q_row_stride, q_head_stride;
    const void* k;
    int64_t k_batch_stride, k_row_stride, k_head_stride;
    const void* v;
    int64_t v_batch_stride, v_row_stride, v_head_stride;
    const void* out;
    int64_t out_batch_stride, out_row_stride, out_head_stride;
    const void* dout;
    int64_t dout_batch_stride, dout_row_stride, dout_head_stride;
    void* dq;
    int64_t dq_batch_stride, dq_row_stride, dq_head_stride;
    void* dk;
    int64_t dk_batch_stride, dk_row_stride, dk_head_stride;
    void* dv;
    int64_t dv_batch_stride, dv_row_stride, dv_head_stride;

    /* softmax_lse: the forward's, (B, H, Sq) fp32 or varlen (H, total_q) fp32.
       softmax_d: output of the same layout, rowsum(dout * out). */
    const float* softmax_lse;
    float* softmax_d;

    const int32_t* cu_seqlens_q;    /* varlen: (B+1,) */
    const int32_t* cu_seqlens_k;    /* varlen: (B+1,) */
    const float* alibi_slopes;      /* (H,) or (B, H) fp32 */
    int64_t alibi_batch_stride;     /* 0 for (H,), H for (B, H) */

    float softmax_scale;
    float softcap;                  /* 0 = off */
    float dropout_p;                /* must be 0 */
    int32_t is_causal;
    int32_t window_size_left;       /* -1 = unbounded */
    int32_t window_size_right;
    int32_t deterministic;          /* accepted; the backward is always deterministic */

    void* workspace;                /* unused: fa_bwd_workspace_size reports 0 */
    size_t workspace_bytes;

    int32_t attention_chunk;        /* as in fa_fwd_params: 0 = off */
} fa_bwd_params;

/* Host-only validation of a backward call (kind: FA_KIND_DENSE or FA_KIND_VARLEN). */
fa_status_t fa_validate_bwd(const fa_bwd_params* p, int32_t kind);

/* Bytes of workspace the backward needs (host-only; currently 0). */
fa_status_t fa_bwd_workspace_size(const fa_bwd_params* p, int32_t kind, size_t* bytes);

/* Backward passes: write dq, dk, dv and softmax_d; enqueue on `stream`.
 * Deterministic: no atomics, every output element is written by one thread. */
fa_status_t fa_mha_bwd(const fa_bwd_params* p, void* stream);
fa_status_t fa_mha_varlen_bwd(const fa_bwd_params* p, void* stream);

/* Thread-local message describing the last non-FA_OK status on this thread. */
const char* fa_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* FA_MI355X_H */
