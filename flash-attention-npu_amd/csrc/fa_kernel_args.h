// fa_kernel_args.h -- the by-value kernel argument blocks (host and device).
//
// Every launch receives one of these structs as its only argument, so the
// host never copies tiling data to the device and never reads device memory
// (the reference copies a tiling struct and a 4 MiB mask H2D and reads
// cache_seqlens back D2H on every call: flash_api.cpp:459,575-580 of
// csrc/arch22/flash_attn_npu_v2).
#pragma once
#include <stdint.h>

namespace fa {

// Strides are in elements; the head dimension is contiguous.
struct FwdArgs {
    const void* q;
    int64_t q_sb, q_si, q_sh;
    const void* k;
    int64_t k_sb, k_si, k_sh;
    const void* v;
    int64_t v_sb, v_si, v_sh;
    void* out;
    int64_t o_sb, o_si, o_sh;
    float* lse;
    int64_t lse_sb, lse_sh;  // (B,H,Sq): b*lse_sb + h*lse_sh + i; varlen (H,T): h*lse_sh + cu_q[b] + i

    const int* seqlens_k;  // per-batch cached length (kvcache), may be null
    const int* cu_seqlens_q;
    const int* cu_seqlens_k;
    const int* block_table;
    const int* batch_idx;
    const float* alibi;
    int64_t bt_stride;
    int64_t alibi_sb;

    float scale;        // softmax_scale
    float scale_log2;   // softmax_scale * log2(e)
    float softcap;      // 0 = off

    int B, Sq, Sk, H, Hk, g;
    int hd;             // head dim present in memory (multiple of 8, <= the kernel's 128;
                        // the dims above it are read as zeros and never written)
    int seqlen_new;     // tokens appended this call (added to seqlens_k)
    int wl, wr;         // normalised window, -1 = unbounded, causal => wr = 0
    int page;           // paged: tokens per block
    int bt_rows;        // paged: rows of the block table (clamp bound)
    int num_blocks;     // paged: rows of the block pool (clamp bound)
    int batch_cache;    // contiguous: rows of the cache (clamp bound for batch_idx)
    int kv_capacity;    // keys addressable per sequence

    // split-KV
    float* part_o;      // [item][BM][Dv] fp32
    float* part_lse;    // [item][BM]
    int* sched;         // [0..B]: item prefix, [B+1..2B]: splits per batch
    int mt_max;         // row tiles per sequence bound
    int page_shift;     // paged: log2(page) when page is a power of two, else -1
    int allow_split;
    int num_splits;     // > 0: forced split count
    int target_items;   // auto split: aim for about this many work items
    int min_chunk;      // auto split: smallest chunk of keys per item
    // decode with a fused append (no rotary): the new tokens (B, S_new, Hk, D)
    const void* k_new;
    int64_t kn_sb, kn_si, kn_sh;
    const void* v_new;
    int64_t vn_sb, vn_si, vn_sh;
    // prefill with rotary: q is rotated as it is loaded (cos/sin: (seqlen_ro, rot_dim/2));
    // rot_cos == nullptr means q is used as stored
    const void* rot_cos;
    const void* rot_sin;
    int rot_dim, rot_interleaved, rot_same_pos, seqlen_ro;
    // kvcache: first valid cache row per sequence (keys are rows leftpad + j);
    // per-sequence new-token counts cu_knew[b+1] - cu_knew[b] (else seqlen_new);
    // rotary position base per sequence (else cache_seqlens)
    const int* leftpad;
    const int* cu_knew;
    const int* rot_pos;
    int chunk;          // attention_chunk, 0 = off
    // FP8 inputs: descale factors per (batch, kv head), null = 1; scores are
    // scaled by qd * kd and the output by vd
    const float* qd;
    const float* kd;
    const float* vd;
    int64_t qd_sb, qd_sh, kd_sb, kd_sh, vd_sb, vd_sh;
    // decode: scores += qv . v (qv like q with the head dim of v), null = off
    const void* qv;
    int64_t qv_sb, qv_si, qv_sh;
    // the kv head of row-tile head hk is hk / kvdiv: 1 when the g query heads
    // of a kv head share its row tiles (Hk, g as given), g when each query
    // head has its own (Hk = H, g = 1)
    int kvdiv;
};

// Backward (dense / varlen). Row layouts as in FwdArgs; lse and dsum share
// one layout: (B,H,Sq): b*lse_sb + h*lse_sh + i; varlen (H,T): h*lse_sh + cu_q[b] + i.
struct BwdArgs {
    const void* q;
    int64_t q_sb, q_si, q_sh;
    const void* k;
    int64_t k_sb, k_si, k_sh;
    const void* v;
    int64_t v_sb, v_si, v_sh;
    const void* out;
    int64_t o_sb, o_si, o_sh;
    const void* dout;
    int64_t do_sb, do_si, do_sh;
    void* dq;
    int64_t dq_sb, dq_si, dq_sh;
    void* dk;
    int64_t dk_sb, dk_si, dk_sh;
    void* dv;
    int64_t dv_sb, dv_si, dv_sh;
    const float* lse;
    float* dsum;        // rowsum(dout * out), written by the dQ kernel (launched first)
    int64_t lse_sb, lse_sh;
    const int* cu_seqlens_q;
    const int* cu_seqlens_k;
    const float* alibi;
    int64_t alibi_sb;
    float scale;        // softmax_scale
    float scale_log2;   // softmax_scale * log2(e)
    float softcap;      // 0 = off
    int B, Sq, Sk, H, Hk, g;
    int hd;             // head dim in memory (<= the kernel's)
    int total_q;        // varlen: rows of q
    int wl, wr;         // normalised window, -1 = unbounded, causal => wr = 0
    int chunk;          // attention_chunk, 0 = off
};

struct KvPrepArgs {
    // new tokens (B, S_new, Hk, D) / (B, S_new, Hk, Dv)
    const void* k_new;
    int64_t kn_sb, kn_si, kn_sh;
    const void* v_new;
    int64_t vn_sb, vn_si, vn_sh;
    void* k_cache;
    int64_t k_sb, k_si, k_sh;
    void* v_cache;
    int64_t v_sb, v_si, v_sh;
    const int* seqlens;
    const int* batch_idx;
    const int* block_table;
    int64_t bt_stride;
    int page, num_blocks, batch_cache, kv_capacity, bt_rows;
    // rotary (cos/sin: (seqlen_ro, rotary_dim/2))
    const void* cos;
    const void* sin;
    int64_t cs_stride;
    int rotary_dim, interleaved, seqlen_ro;
    // q rotation (decode): q (B, Sq, H, D) -> q_out (B, Sq, H, D) contiguous; null = none
    const void* q;
    int64_t q_sb, q_si, q_sh;
    void* q_out;
    int q_same_pos;
    int B, S_new, Sq, H, Hk, D, Dv;
    // ragged layouts: new tokens (total_new, Hk, D) split by cu_knew, q
    // (total_q, H, D) split by cu_q; rotary position base per sequence
    const int* cu_knew;
    const int* cu_q;
    const int* rot_pos;
    int total_new, total_q;
};

}  // namespace fa
