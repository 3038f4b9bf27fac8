// fa_api.cpp -- host side of the C ABI declared in include/fa_mi355x.h:
// validation, split-KV planning, workspace layout and kernel launches.
//
// Mirrors the checks and decisions of the reference host code
// (csrc/arch22/flash_attn_npu_v2/flash_api.cpp: mha_fwd_kvcache :356-626,
// mha_fwd :628-826, mha_varlen_fwd :828-1060; csrc/arch22/flash_attn_npu_v3/
// flash_api.cpp: mha_fwd :60-491) without its host round trips: the plan is a
// function of host-known shapes only, and the per-sequence split is decided on
// the device from cache_seqlens.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>
#include <type_traits>

#include "../../include/fa_mi355x.h"
#include "fa_kernel_args.h"

namespace fa {
int fwd_tile_rows(int d);
int fwd_tile_keys(int d);
int decode_workers(int cus);
hipError_t launch_fwd(const FwdArgs& a, int dtype, int d, int grid, hipStream_t stream);
hipError_t launch_merge(const FwdArgs& a, int dtype, int d, hipStream_t stream);
hipError_t launch_decode(const FwdArgs& a, int dtype, int d, int grid, hipStream_t stream);
hipError_t launch_decode_merge(const FwdArgs& a, int dtype, int d, int grid, hipStream_t stream);
hipError_t launch_combine_flat(const float* po, const float* pl, int S, int64_t R, int Dv, void* out, int64_t ors,
                               int out_dtype, float* lse, hipStream_t stream);
hipError_t launch_kv_prep(const KvPrepArgs& a, int dtype, hipStream_t stream);
hipError_t launch_bwd(const BwdArgs& a, int dtype, int d, int grid_kv, int grid_q, hipStream_t stream);
int bwd_key_block(int d);
int bwd_row_block(int d);
}  // namespace fa

namespace {

constexpr int kMaxBatch = 2048;   // sequences per attention launch (per-batch plans live in LDS)
constexpr int kDecodeRows = 16;   // rows per (b, kv head) that take the decode kernel

thread_local std::string g_err;

fa_status_t fail(fa_status_t st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return st;
}

#define FA_CHECK(cond, ...)                              \
    do {                                                 \
        if (!(cond)) return fail(FA_EINVAL, __VA_ARGS__); \
    } while (0)

int cu_count() {
    static std::mutex mu;
    static int counts[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    std::lock_guard<std::mutex> lk(mu);
    if (counts[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        counts[dev] = n;
    }
    return counts[dev];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool strides8(int64_t a, int64_t b, int64_t c) { return (a % 8) == 0 && (b % 8) == 0 && (c % 8) == 0; }
bool strides16(int64_t a, int64_t b, int64_t c) { return (a % 16) == 0 && (b % 16) == 0 && (c % 16) == 0; }

struct Plan {
    bool decode;
    int BM, BN;
    int g;
    int hk_eff;         // heads that own row tiles: nheads_k, or nheads without GQA packing
    int rows_max;       // packed rows per (b, kv head) bound
    int mt_max;
    int kv_capacity;
    bool allow_split;
    int target_items;
    int min_chunk;
    int64_t items_max;  // bound on work items (partial buffer size)
    int grid;
    bool rotary;
    int workers;        // decode: wave workers
    int kd;             // kernel head dim (64, 128 or 256)
    size_t off_sched, off_plse, off_po, off_qrot, total;
};

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

fa_status_t validate(const fa_fwd_params* p, int kind) {
    FA_CHECK(p != nullptr, "params must not be null");
    FA_CHECK(p->abi_version == FA_MI355X_ABI_VERSION, "abi_version %d does not match library ABI %d", p->abi_version,
             FA_MI355X_ABI_VERSION);
    FA_CHECK(kind == FA_KIND_KVCACHE || kind == FA_KIND_DENSE || kind == FA_KIND_VARLEN, "unknown kind %d", kind);
    const bool f8 = p->dtype == FA_DTYPE_FP8_E4M3;
    FA_CHECK(p->dtype == FA_DTYPE_FP16 || p->dtype == FA_DTYPE_BF16 || f8,
             "FlashAttention only support fp16 and bf16 data type (and fp8 e4m3 inputs in the forward)");
    FA_CHECK(p->batch >= 1, "batch size must be positive");
    if (f8) {
        // 16-byte loads of e4m3 rows: 16-element head-dim chunks and row starts
        FA_CHECK(p->headdim % 16 == 0, "FP8 inputs need a head dimension that is a multiple of 16");
        FA_CHECK(strides16(p->q_batch_stride, p->q_row_stride, p->q_head_stride) &&
                     strides16(p->k_batch_stride, p->k_row_stride, p->k_head_stride) &&
                     strides16(p->v_batch_stride, p->v_row_stride, p->v_head_stride),
                 "FP8 q, k and v strides must be multiples of 16 elements");
        FA_CHECK(p->rotary_cos == nullptr && p->rotary_sin == nullptr, "rotary is not supported with FP8 inputs");
        if (p->k_new)
            FA_CHECK(strides16(p->knew_batch_stride, p->knew_row_stride, p->knew_head_stride) &&
                         strides16(p->vnew_batch_stride, p->vnew_row_stride, p->vnew_head_stride),
                     "FP8 k and v strides must be multiples of 16 elements");
    }
    FA_CHECK(p->nheads >= 1 && p->nheads_k >= 1, "number of heads must be positive");
    FA_CHECK(p->nheads % p->nheads_k == 0, "Number of heads in key/value must divide number of heads in query");
    FA_CHECK(p->headdim >= 1, "head dimension must be positive");
    if (p->qv) {
        FA_CHECK(!f8, "qv is not supported with FP8 inputs");
        FA_CHECK(aligned16(p->qv) && strides8(p->qv_batch_stride, p->qv_row_stride, p->qv_head_stride),
                 "qv must be 16-byte aligned with strides that are multiples of 8 elements");
        const int64_t rows = (int64_t)p->seqlen_q * (p->no_pack_gqa ? 1 : p->nheads / p->nheads_k);
        if (rows > kDecodeRows || p->headdim > 128)
            return fail(FA_EUNSUPPORTED,
                        "qv is supported where the decode kernel runs: at most %d query rows per kv head "
                        "(seqlen_q * nheads / nheads_k) and headdim <= 128",
                        kDecodeRows);
    }
    FA_CHECK(p->headdim % 8 == 0, "head dimension must be a multiple of 8");
    FA_CHECK(p->headdim <= 256, "FlashAttention only supports head dimension at most 256");
    FA_CHECK(p->headdim_v == p->headdim, "headdim_v (%d) must equal headdim (%d)", p->headdim_v, p->headdim);
    if (p->dropout_p != 0.f) return fail(FA_EUNSUPPORTED, "dropout is not supported (forward inference only)");
    FA_CHECK(p->softcap >= 0.f, "softcap must be >= 0");
    FA_CHECK(p->num_splits >= 0, "num_splits must be >= 0");
    FA_CHECK(p->attention_chunk >= 0, "attention_chunk must be >= 0");
    FA_CHECK(p->seqlen_q >= 0, "seqlen_q must be >= 0");
    // packed rows (query position x q head of one kv head) are 32-bit indices in the kernels
    FA_CHECK((int64_t)p->seqlen_q * (p->nheads / p->nheads_k) <= (int64_t)1 << 30,
             "seqlen_q * (nheads / nheads_k) must be at most 2^30");
    // key indices (and tile counts rounded up from them) are 32-bit in the kernels
    FA_CHECK(p->seqlen_k <= (1 << 30), "seqlen_k must be at most 2^30");
    FA_CHECK(p->block_table == nullptr || (int64_t)p->max_blocks_per_seq * p->page_block_size <= (int64_t)1 << 30,
             "block_table columns x page_block_size must be at most 2^30");
    // a call with no query rows (it may still append k / v) may pass empty,
    // null q / out / softmax_lse, as zero-size tensors have no storage
    const int64_t q_rows = p->cu_seqlens_q ? p->total_q : (int64_t)p->batch * p->seqlen_q;
    FA_CHECK(p->k && p->v && (q_rows == 0 || (p->q && p->out && p->softmax_lse)),
             "q, k, v, out and softmax_lse must be given");
    FA_CHECK(aligned16(p->q) && aligned16(p->k) && aligned16(p->v) && aligned16(p->out),
             "q, k, v and out must be 16-byte aligned");
    FA_CHECK(strides8(p->q_batch_stride, p->q_row_stride, p->q_head_stride), "q strides must be multiples of 8 elements");
    FA_CHECK(strides8(p->k_batch_stride, p->k_row_stride, p->k_head_stride), "k strides must be multiples of 8 elements");
    FA_CHECK(strides8(p->v_batch_stride, p->v_row_stride, p->v_head_stride), "v strides must be multiples of 8 elements");
    FA_CHECK(strides8(p->out_batch_stride, p->out_row_stride, p->out_head_stride),
             "out strides must be multiples of 8 elements");
    if (p->alibi_slopes)
        FA_CHECK(p->alibi_batch_stride == 0 || p->alibi_batch_stride == p->nheads,
                 "alibi_slopes must have shape (nheads) or (batch_size, nheads)");
    if (kind == FA_KIND_KVCACHE) {
        const bool paged = p->block_table != nullptr;
        if (paged) {
            FA_CHECK(p->page_block_size >= 1, "page_block_size must be positive");
            FA_CHECK(p->max_blocks_per_seq >= 1, "block_table must have at least one column");
            FA_CHECK(p->batch_cache >= 1, "paged KV cache must have at least one block");
            FA_CHECK(p->block_table_rows >= (p->cache_batch_idx ? 1 : p->batch), "block_table must have a row per batch entry");
        } else {
            FA_CHECK(p->batch_cache >= 1, "k_cache batch must be positive");
            FA_CHECK(p->seqlen_k >= 1, "k_cache seqlen must be positive");
            if (!p->cache_batch_idx)
                FA_CHECK(p->batch_cache >= p->batch, "k_cache batch (%d) smaller than q batch (%d) without cache_batch_idx",
                         p->batch_cache, p->batch);
        }
        FA_CHECK((p->k_new == nullptr) == (p->v_new == nullptr), "If key is supplied, value must also be passed in");
        if (p->cache_leftpad)
            FA_CHECK(!paged, "cache_leftpad is not supported with a paged KV cache (page_table / block_table)");
        if (p->cu_seqlens_q) FA_CHECK(p->total_q >= 0, "total_q must be >= 0 with cu_seqlens_q");
        if (p->cu_seqlens_k_new) {
            FA_CHECK(p->k_new != nullptr, "cu_seqlens_k_new is given without new keys k / v");
            FA_CHECK(p->total_k_new >= 0, "total_k_new must be >= 0 with cu_seqlens_k_new");
        }
        if (p->k_new) {
            FA_CHECK(p->cu_seqlens_k_new || p->seqlen_new >= 1, "k/v must have at least one new token");
            FA_CHECK(p->cache_seqlens != nullptr, "cache_seqlens is required to append k/v");
            FA_CHECK(aligned16(p->k_new) && aligned16(p->v_new), "k and v must be 16-byte aligned");
            FA_CHECK(strides8(p->knew_batch_stride, p->knew_row_stride, p->knew_head_stride) &&
                         strides8(p->vnew_batch_stride, p->vnew_row_stride, p->vnew_head_stride),
                     "k and v strides must be multiples of 8 elements");
        }
        if (p->rotary_cos || p->rotary_sin) {
            FA_CHECK(p->rotary_cos && p->rotary_sin, "rotary_cos and rotary_sin must be given together");
            FA_CHECK(p->k_new != nullptr, "If rotary cos/sin are provided, new key / value to be appended to KV cache must also be provided");
            FA_CHECK(p->rotary_dim > 0 && p->rotary_dim % 16 == 0, "rotary_dim must be divisible by 16");
            FA_CHECK(p->rotary_dim <= p->headdim, "rotary_dim must be <= headdim");
            FA_CHECK(p->seqlen_ro >= 1, "rotary_cos must have at least one row");
            FA_CHECK((reinterpret_cast<uintptr_t>(p->rotary_cos) & 7u) == 0 &&
                         (reinterpret_cast<uintptr_t>(p->rotary_sin) & 7u) == 0,
                     "rotary_cos/sin must be 8-byte aligned");
        }
    } else {
        FA_CHECK(p->k_new == nullptr && p->v_new == nullptr, "k_new/v_new are only valid for the kvcache forward");
        FA_CHECK(!p->cache_leftpad && !p->cu_seqlens_k_new && !p->rotary_seqlens,
                 "cache_leftpad, cu_seqlens_k_new and rotary_seqlens are only valid for the kvcache forward");
        FA_CHECK(p->rotary_cos == nullptr && p->rotary_sin == nullptr, "rotary is only valid for the kvcache forward");
        FA_CHECK(p->block_table == nullptr || kind == FA_KIND_VARLEN, "block_table is not valid for the dense forward");
        FA_CHECK(p->seqlen_k >= 0, "seqlen_k must be >= 0");
        if (kind == FA_KIND_VARLEN) {
            FA_CHECK(p->cu_seqlens_q != nullptr, "cu_seqlens_q is required");
            FA_CHECK(p->cu_seqlens_k || (p->block_table && p->cache_seqlens),
                     "cu_seqlens_k is required (or, with a block_table, seqused_k)");
            FA_CHECK(p->total_q >= 0, "total_q must be >= 0");
            if (p->block_table) {
                FA_CHECK(p->page_block_size >= 1 && p->max_blocks_per_seq >= 1 && p->batch_cache >= 1,
                         "paged varlen needs page_block_size, block_table columns and num_blocks");
            }
        }
    }
    return FA_OK;
}

void make_plan(const fa_fwd_params* p, int kind, Plan& pl) {
    pl.hk_eff = p->no_pack_gqa ? p->nheads : p->nheads_k;
    pl.g = p->nheads / pl.hk_eff;
    pl.rows_max = p->seqlen_q * pl.g;
    // kernel head dim: the prefill kernels come at 64, 128 and 256, the
    // decode kernel at 64 and 128; each serves the head dims up to its own
    // (the dims above the real ones read as zero); decode shapes above 128
    // run on the prefill kernel. A forced split count (num_splits >= 1) also
    // runs on the prefill kernel, which cuts each sequence's keys into
    // exactly that many chunks (1: none), as the reference's fixed split
    // does (csrc/arch22/flash_attn_npu_v3/fa_split.h:335-402); the decode
    // kernel's stream-K split is the heuristic one (num_splits = 0). Calls
    // with qv stay on the decode kernel whatever num_splits says: only it
    // forms the qv term.
    pl.decode = pl.rows_max <= kDecodeRows && p->headdim <= 128 && (p->num_splits == 0 || p->qv != nullptr);
    pl.kd = p->headdim <= 64 ? 64 : p->headdim <= 128 ? 128 : 256;
    pl.BM = pl.decode ? kDecodeRows : fa::fwd_tile_rows(pl.kd);
    pl.BN = pl.decode ? 32 : fa::fwd_tile_keys(pl.kd);
    pl.mt_max = (pl.rows_max + pl.BM - 1) / pl.BM;
    if (pl.mt_max < 1) pl.mt_max = 1;
    if (kind == FA_KIND_KVCACHE) {
        pl.kv_capacity = p->block_table ? (int)std::min<int64_t>((int64_t)p->max_blocks_per_seq * p->page_block_size, INT_MAX)
                                        : p->seqlen_k;
    } else if (kind == FA_KIND_VARLEN) {
        pl.kv_capacity = p->block_table ? (int)std::min<int64_t>((int64_t)p->max_blocks_per_seq * p->page_block_size, INT_MAX)
                                        : INT_MAX;
    } else {
        pl.kv_capacity = p->seqlen_k;
    }
    const int cus = cu_count();
    pl.rotary = kind == FA_KIND_KVCACHE && p->rotary_cos != nullptr;
    // batch entries per attention launch (larger batches run in chunks)
    const int pb = std::min(p->batch, kMaxBatch);
    size_t off = 0;
    pl.off_sched = off;
    off = align256(off + sizeof(int) * (2 * (size_t)pb + 2));
    if (pl.decode) {
        // stream-K decode: one workgroup of 4 wave workers per CU, <= 2 partials per worker
        pl.grid = cus;
        pl.workers = fa::decode_workers(cus);
        pl.allow_split = true;
        pl.items_max = (int64_t)pl.workers * 2;
        pl.target_items = 0;
        pl.min_chunk = 0;
    } else {
        const int occ = 2;  // prefill workgroups per CU
        const int64_t base_bound = (int64_t)pb * pl.hk_eff * pl.mt_max;
        pl.workers = 0;
        pl.target_items = 2 * cus;
        pl.min_chunk = 2 * pl.BN;
        if (p->num_splits == 1) pl.allow_split = false;
        else if (p->num_splits > 1) pl.allow_split = true;
        else pl.allow_split = base_bound < cus;
        if (!pl.allow_split) pl.items_max = base_bound;
        else if (p->num_splits > 1) pl.items_max = base_bound * p->num_splits;
        else pl.items_max = base_bound + pl.target_items;
        // Without a split, sequences of one length (no cu_seqlens_q) run on
        // one workgroup per CU that takes several items, paired heavy with
        // light by the kernel's alternating passes: no workgroup start-up per
        // item (1-4.5 % faster than 2 workgroups per CU on dense shapes).
        // Ragged query lengths keep one workgroup per item, which the hardware
        // hands out heaviest first as CUs free up.
        if (pl.allow_split) pl.grid = (int)std::min<int64_t>(pl.items_max, (int64_t)occ * cus);
        else if (!p->cu_seqlens_q) pl.grid = (int)std::min<int64_t>(pl.items_max, (int64_t)cus);
        else pl.grid = (int)std::min<int64_t>(pl.items_max, INT_MAX);
        if (pl.grid < 1) pl.grid = 1;
    }
    pl.off_plse = off;
    if (pl.allow_split) off = align256(off + sizeof(float) * (size_t)pl.items_max * pl.BM);
    pl.off_po = off;
    // partial rows are written at the kernel's head dim
    if (pl.allow_split) off = align256(off + sizeof(float) * (size_t)pl.items_max * pl.BM * pl.kd);
    pl.off_qrot = off;
    // decode reads a rotated copy of q; prefill rotates q as it loads it
    const int64_t q_rows = (kind == FA_KIND_KVCACHE && p->cu_seqlens_q) ? p->total_q : (int64_t)p->batch * p->seqlen_q;
    if (pl.rotary && pl.decode) off = align256(off + 2 * (size_t)q_rows * p->nheads * p->headdim);
    pl.total = off;
}

// Byte offset of batch entry b0 in a batch-strided tensor of esz-byte elements.
template <typename T>
T* boff(T* ptr, int64_t b0, int64_t stride, int esz) {
    if (!ptr) return ptr;
    using B = std::conditional_t<std::is_const<T>::value, const char, char>;
    return reinterpret_cast<T*>(reinterpret_cast<B*>(ptr) + b0 * stride * esz);
}

// The forward. ws / ws_bytes: the scratch the kernels use (the caller's
// workspace, or the library's static scratch for the no-allocation entry
// point). Per-batch kernel plans live in LDS, so a call with more than
// kMaxBatch sequences runs its attention as consecutive launches over batch
// chunks on the same stream (the KV append runs once, for the whole batch,
// before them); the chunks reuse one workspace, since each chunk's merge
// precedes the next chunk's attention on the stream.
fa_status_t run_forward_ws(const fa_fwd_params* p, int kind, void* stream_v, void* ws_v, size_t ws_bytes) {
    fa_status_t st = validate(p, kind);
    if (st != FA_OK) return st;
    hipStream_t stream = static_cast<hipStream_t>(stream_v);
    Plan pl;
    make_plan(p, kind, pl);
    if (pl.total > 0) {
        if (!ws_v || ws_bytes < pl.total)
            return fail(FA_EWORKSPACE, "workspace of %zu bytes required, %zu given", pl.total, ws_v ? ws_bytes : (size_t)0);
        if (reinterpret_cast<uintptr_t>(ws_v) & 255u) return fail(FA_EWORKSPACE, "workspace must be 256-byte aligned");
    }
    char* ws = static_cast<char*>(ws_v);
    const bool paged = p->block_table != nullptr;
    const bool f8 = p->dtype == FA_DTYPE_FP8_E4M3;
    const int esz = f8 ? 1 : 2;  // bytes per q / k / v element (out is 16-bit)
    const bool chunked = p->batch > kMaxBatch;

    const void* q_ptr = p->q;
    int64_t q_sb = p->q_batch_stride, q_si = p->q_row_stride, q_sh = p->q_head_stride;
    int q_esz = esz;

    auto mark = [&](int i) {
        if (p->stage_events && p->stage_events[i]) (void)hipEventRecord(static_cast<hipEvent_t>(p->stage_events[i]), stream);
    };
    mark(0);
    // Decode without rotary appends inside the attention kernel; otherwise the
    // append (with the key rotation, and for decode the q rotation) runs as
    // its own launch first. Prefill rotates q inside its q load. The decode
    // kernel visits only the key tiles some query row sees and writes a new
    // token from the tile that holds it, so the fused append is used only
    // where every new token lies in a visited tile: at most seqlen_q new
    // tokens (the first row sees its own diagonal key), or no left window and
    // no attention chunk (every tile from key 0 is visited); ragged q (a
    // sequence may have no query rows, hence no tiles) takes the separate
    // append, as does a batch run in chunks, and a call with no query rows
    // (it launches no attention kernel at all).
    const bool local_left = p->window_size_left >= 0 || p->attention_chunk > 0;
    const bool fused_append = kind == FA_KIND_KVCACHE && p->k_new && pl.decode && !pl.rotary && !p->cu_seqlens_k_new &&
                              !p->cu_seqlens_q && !chunked && !p->no_pack_gqa && p->seqlen_q > 0 &&
                              (p->seqlen_new <= p->seqlen_q || !local_left);
    if (kind == FA_KIND_KVCACHE && p->k_new && !fused_append) {
        fa::KvPrepArgs k{};
        k.k_new = p->k_new;
        k.kn_sb = p->knew_batch_stride;
        k.kn_si = p->knew_row_stride;
        k.kn_sh = p->knew_head_stride;
        k.v_new = p->v_new;
        k.vn_sb = p->vnew_batch_stride;
        k.vn_si = p->vnew_row_stride;
        k.vn_sh = p->vnew_head_stride;
        k.k_cache = p->k;
        k.k_sb = p->k_batch_stride;
        k.k_si = p->k_row_stride;
        k.k_sh = p->k_head_stride;
        k.v_cache = p->v;
        k.v_sb = p->v_batch_stride;
        k.v_si = p->v_row_stride;
        k.v_sh = p->v_head_stride;
        k.seqlens = p->cache_seqlens;
        k.batch_idx = p->cache_batch_idx;
        k.block_table = p->block_table;
        k.bt_stride = p->block_table_batch_stride;
        k.page = paged ? p->page_block_size : 1;
        k.bt_rows = p->block_table_rows;
        k.num_blocks = paged ? p->batch_cache : 0;
        k.batch_cache = p->batch_cache;
        k.kv_capacity = pl.kv_capacity;
        k.cos = p->rotary_cos;
        k.sin = p->rotary_sin;
        k.cs_stride = p->rotary_dim / 2;
        k.rotary_dim = pl.rotary ? p->rotary_dim : 0;
        k.interleaved = p->rotary_interleaved;
        k.seqlen_ro = p->seqlen_ro;
        k.q = p->q;
        k.q_sb = p->q_batch_stride;
        k.q_si = p->q_row_stride;
        k.q_sh = p->q_head_stride;
        k.q_out = pl.rotary && pl.decode && p->seqlen_q > 0 ? ws + pl.off_qrot : nullptr;
        const bool local = p->window_size_left >= 0 || p->window_size_right >= 0;
        k.q_same_pos = !(p->is_causal || local);
        k.B = p->batch;
        k.S_new = p->seqlen_new;
        k.Sq = p->seqlen_q;
        k.H = p->nheads;
        k.Hk = p->nheads_k;
        k.D = p->headdim;
        k.Dv = p->headdim_v;
        k.cu_knew = p->cu_seqlens_k_new;
        k.total_new = p->cu_seqlens_k_new ? p->total_k_new : 0;
        k.cu_q = p->cu_seqlens_q;
        k.total_q = p->cu_seqlens_q ? p->total_q : 0;
        k.rot_pos = pl.rotary ? p->rotary_seqlens : nullptr;
        hipError_t e = fa::launch_kv_prep(k, p->dtype, stream);
        if (e != hipSuccess) return fail(FA_EHIP, "kv_prep launch failed: %s", hipGetErrorString(e));
        if (k.q_out) {
            q_ptr = ws + pl.off_qrot;
            q_sh = p->headdim;
            q_si = (int64_t)p->nheads * p->headdim;
            q_sb = (int64_t)p->seqlen_q * q_si;
            q_esz = 2;
        }
    }
    // no query rows: the append above is all the work
    if ((p->seqlen_q == 0 && kind != FA_KIND_VARLEN) || (p->cu_seqlens_q && p->total_q == 0)) {
        mark(1);
        mark(2);
        mark(3);
        return FA_OK;
    }

    const bool ragged_q = kind == FA_KIND_VARLEN || (kind == FA_KIND_KVCACHE && p->cu_seqlens_q);
    const bool kv_batched = !paged && !p->cache_batch_idx && !(kind == FA_KIND_VARLEN && p->cu_seqlens_k);
    mark(1);
    for (int64_t b0 = 0; b0 < p->batch; b0 += kMaxBatch) {
        const int nb = (int)std::min<int64_t>(kMaxBatch, p->batch - b0);
        fa::FwdArgs a{};
        a.q = ragged_q ? q_ptr : boff(q_ptr, b0, q_sb, q_esz);
        a.q_sb = q_sb;
        a.q_si = q_si;
        a.q_sh = q_sh;
        a.k = kv_batched ? boff(p->k, b0, p->k_batch_stride, esz) : p->k;
        a.k_sb = p->k_batch_stride;
        a.k_si = p->k_row_stride;
        a.k_sh = p->k_head_stride;
        a.v = kv_batched ? boff(p->v, b0, p->v_batch_stride, esz) : p->v;
        a.v_sb = p->v_batch_stride;
        a.v_si = p->v_row_stride;
        a.v_sh = p->v_head_stride;
        a.out = ragged_q ? p->out : boff(p->out, b0, p->out_batch_stride, 2);
        a.o_sb = p->out_batch_stride;
        a.o_si = p->out_row_stride;
        a.o_sh = p->out_head_stride;
        if (ragged_q) {
            a.lse = p->softmax_lse;
            a.lse_sb = 0;
            a.lse_sh = p->total_q;
        } else {
            a.lse_sb = (int64_t)p->nheads * p->seqlen_q;
            a.lse_sh = p->seqlen_q;
            a.lse = p->softmax_lse + (int64_t)b0 * a.lse_sb;
        }
        auto at = [&](const int32_t* x) { return x ? x + b0 : x; };
        a.seqlens_k = kind == FA_KIND_DENSE ? nullptr : at(p->cache_seqlens);  // kvcache lengths / varlen seqused_k
        a.cu_seqlens_q = ragged_q ? at(p->cu_seqlens_q) : nullptr;  // prefix values stay absolute row offsets
        a.cu_seqlens_k = kind == FA_KIND_VARLEN ? at(p->cu_seqlens_k) : nullptr;
        a.batch_idx = kind == FA_KIND_KVCACHE ? at(p->cache_batch_idx) : nullptr;
        const bool bt_batched = paged && !a.batch_idx;
        a.block_table = bt_batched ? p->block_table + (int64_t)b0 * p->block_table_batch_stride : p->block_table;
        a.bt_stride = p->block_table_batch_stride;
        a.bt_rows = bt_batched ? p->block_table_rows - b0 : p->block_table_rows;
        a.alibi = p->alibi_slopes ? p->alibi_slopes + (int64_t)b0 * p->alibi_batch_stride : nullptr;
        a.alibi_sb = p->alibi_batch_stride;
        a.scale = p->softmax_scale;
        a.scale_log2 = p->softmax_scale * 1.4426950408889634f;
        a.softcap = p->softcap;
        a.B = nb;
        a.Sq = p->seqlen_q;
        a.Sk = kind == FA_KIND_KVCACHE ? pl.kv_capacity : p->seqlen_k;
        a.H = p->nheads;
        a.Hk = pl.hk_eff;
        a.g = pl.g;
        a.kvdiv = pl.hk_eff / p->nheads_k;
        a.qv = ragged_q || !p->qv ? p->qv : boff(p->qv, b0, p->qv_batch_stride, 2);
        a.qv_sb = p->qv_batch_stride;
        a.qv_si = p->qv_row_stride;
        a.qv_sh = p->qv_head_stride;
        a.hd = p->headdim;
        a.seqlen_new = (kind == FA_KIND_KVCACHE && p->k_new && !p->cu_seqlens_k_new) ? p->seqlen_new : 0;
        if (kind == FA_KIND_KVCACHE) {
            a.leftpad = at(p->cache_leftpad);
            a.cu_knew = p->k_new ? at(p->cu_seqlens_k_new) : nullptr;
            a.rot_pos = pl.rotary ? at(p->rotary_seqlens) : nullptr;
        }
        a.chunk = p->attention_chunk;
        if (f8) {  // descales are read for FP8 inputs only
            a.qd = p->q_descale ? p->q_descale + (int64_t)b0 * p->q_descale_batch_stride : nullptr;
            a.qd_sb = p->q_descale_batch_stride;
            a.qd_sh = p->q_descale_head_stride;
            a.kd = p->k_descale ? p->k_descale + (int64_t)b0 * p->k_descale_batch_stride : nullptr;
            a.kd_sb = p->k_descale_batch_stride;
            a.kd_sh = p->k_descale_head_stride;
            a.vd = p->v_descale ? p->v_descale + (int64_t)b0 * p->v_descale_batch_stride : nullptr;
            a.vd_sb = p->v_descale_batch_stride;
            a.vd_sh = p->v_descale_head_stride;
        }
        if (fused_append) {  // one chunk only
            a.k_new = p->k_new;
            a.kn_sb = p->knew_batch_stride;
            a.kn_si = p->knew_row_stride;
            a.kn_sh = p->knew_head_stride;
            a.v_new = p->v_new;
            a.vn_sb = p->vnew_batch_stride;
            a.vn_si = p->vnew_row_stride;
            a.vn_sh = p->vnew_head_stride;
        }
        if (pl.rotary && !pl.decode) {
            a.rot_cos = p->rotary_cos;
            a.rot_sin = p->rotary_sin;
            a.rot_dim = p->rotary_dim;
            a.rot_interleaved = p->rotary_interleaved ? 1 : 0;
            a.rot_same_pos = !(p->is_causal || p->window_size_left >= 0 || p->window_size_right >= 0);
            a.seqlen_ro = p->seqlen_ro;
        }
        // window normalisation (flash_api.cpp:483-494): the seqlen-dependent rules
        // leave the mask unchanged, causal forces the right edge to the diagonal
        int wl = p->window_size_left < 0 ? -1 : p->window_size_left;
        int wr = p->window_size_right < 0 ? -1 : p->window_size_right;
        if (p->is_causal) wr = 0;
        a.wl = wl;
        a.wr = wr;
        a.page = paged ? p->page_block_size : 1;
        a.num_blocks = paged ? p->batch_cache : 0;
        a.batch_cache = kind == FA_KIND_KVCACHE ? (kv_batched ? p->batch_cache - b0 : p->batch_cache) : nb;
        a.kv_capacity = pl.kv_capacity;
        a.part_o = pl.allow_split ? reinterpret_cast<float*>(ws + pl.off_po) : nullptr;
        a.part_lse = pl.allow_split ? reinterpret_cast<float*>(ws + pl.off_plse) : nullptr;
        a.sched = reinterpret_cast<int*>(ws + pl.off_sched);
        a.allow_split = pl.allow_split ? 1 : 0;
        a.num_splits = p->num_splits > 1 ? p->num_splits : 0;
        a.target_items = pl.target_items;
        a.min_chunk = pl.min_chunk;
        a.mt_max = pl.mt_max;
        a.page_shift = -1;
        if (paged && (p->page_block_size & (p->page_block_size - 1)) == 0) {
            int sh = 0;
            while ((1 << sh) < p->page_block_size) ++sh;
            a.page_shift = sh;
        }

        hipError_t e = pl.decode ? fa::launch_decode(a, p->dtype, pl.kd, pl.grid, stream)
                                 : fa::launch_fwd(a, p->dtype, pl.kd, pl.grid, stream);
        if (e != hipSuccess) return fail(FA_EHIP, "attention launch failed: %s", hipGetErrorString(e));
        if (b0 + nb >= p->batch) mark(2);
        if (pl.decode) {
            hipError_t em = fa::launch_decode_merge(a, p->dtype, pl.kd, pl.grid, stream);
            if (em != hipSuccess) return fail(FA_EHIP, "merge launch failed: %s", hipGetErrorString(em));
        } else if (pl.allow_split) {
            hipError_t em = fa::launch_merge(a, p->dtype, pl.kd, stream);
            if (em != hipSuccess) return fail(FA_EHIP, "merge launch failed: %s", hipGetErrorString(em));
        }
    }
    mark(3);
    return FA_OK;
}

fa_status_t run_forward(const fa_fwd_params* p, int kind, void* stream_v) {
    if (!p) return fail(FA_EINVAL, "params must not be null");
    return run_forward_ws(p, kind, stream_v, p->workspace, p->workspace ? p->workspace_bytes : 0);
}

// ---- backward ---------------------------------------------------------------------------
// Checks of mha_bwd / mha_varlen_bwd (flash_api.cpp:1063-1299 of the reference),
// with this build's layout rules (16-byte rows, strides in multiples of 8).
fa_status_t validate_bwd(const fa_bwd_params* p, int kind) {
    FA_CHECK(p != nullptr, "params must not be null");
    FA_CHECK(p->abi_version == FA_MI355X_ABI_VERSION, "abi_version %d does not match library ABI %d", p->abi_version,
             FA_MI355X_ABI_VERSION);
    FA_CHECK(kind == FA_KIND_DENSE || kind == FA_KIND_VARLEN, "backward kind must be dense or varlen, got %d", kind);
    FA_CHECK(p->dtype == FA_DTYPE_FP16 || p->dtype == FA_DTYPE_BF16,
             "FlashAttention only support fp16 and bf16 data type");
    FA_CHECK(p->batch >= 1, "batch size must be positive");
    FA_CHECK(p->nheads >= 1 && p->nheads_k >= 1, "number of heads must be positive");
    FA_CHECK(p->nheads % p->nheads_k == 0, "Number of heads in key/value must divide number of heads in query");
    FA_CHECK(p->headdim >= 1 && p->headdim % 8 == 0, "head dimension must be a positive multiple of 8");
    FA_CHECK(p->headdim <= 256, "FlashAttention only supports head dimension at most 256");
    if (p->dropout_p != 0.f) return fail(FA_EUNSUPPORTED, "dropout is not supported");
    FA_CHECK(p->softcap >= 0.f, "softcap must be non-negative (0.0 disables softcap)");
    FA_CHECK(p->attention_chunk >= 0, "attention_chunk must be >= 0");
    FA_CHECK(p->seqlen_q >= 0 && p->seqlen_k >= 0, "sequence lengths must be >= 0");
    FA_CHECK((int64_t)p->seqlen_q * (p->nheads / p->nheads_k) <= (int64_t)1 << 30,
             "seqlen_q * (nheads / nheads_k) must be at most 2^30");
    FA_CHECK(p->seqlen_k <= (1 << 30), "seqlen_k must be at most 2^30");
    FA_CHECK(p->q && p->k && p->v && p->out && p->dout && p->dq && p->dk && p->dv,
             "q, k, v, out, dout, dq, dk and dv must be given");
    FA_CHECK(p->softmax_lse && p->softmax_d, "softmax_lse and softmax_d must be given");
    FA_CHECK(aligned16(p->q) && aligned16(p->k) && aligned16(p->v) && aligned16(p->out) && aligned16(p->dout) &&
                 aligned16(p->dq) && aligned16(p->dk) && aligned16(p->dv),
             "q, k, v, out, dout, dq, dk and dv must be 16-byte aligned");
    FA_CHECK(strides8(p->q_batch_stride, p->q_row_stride, p->q_head_stride) &&
                 strides8(p->k_batch_stride, p->k_row_stride, p->k_head_stride) &&
                 strides8(p->v_batch_stride, p->v_row_stride, p->v_head_stride) &&
                 strides8(p->out_batch_stride, p->out_row_stride, p->out_head_stride) &&
                 strides8(p->dout_batch_stride, p->dout_row_stride, p->dout_head_stride) &&
                 strides8(p->dq_batch_stride, p->dq_row_stride, p->dq_head_stride) &&
                 strides8(p->dk_batch_stride, p->dk_row_stride, p->dk_head_stride) &&
                 strides8(p->dv_batch_stride, p->dv_row_stride, p->dv_head_stride),
             "strides must be multiples of 8 elements");
    if (p->alibi_slopes)
        FA_CHECK(p->alibi_batch_stride == 0 || p->alibi_batch_stride == p->nheads,
                 "alibi_slopes must have shape (nheads) or (batch_size, nheads)");
    if (kind == FA_KIND_VARLEN) {
        FA_CHECK(p->cu_seqlens_q && p->cu_seqlens_k, "cu_seqlens_q and cu_seqlens_k are required for varlen");
        FA_CHECK(p->total_q >= 0, "total_q must be >= 0");
    } else {
        FA_CHECK(!p->cu_seqlens_q && !p->cu_seqlens_k, "cu_seqlens are only valid for varlen");
    }
    return FA_OK;
}

// Like the forward, a batch above kMaxBatch runs as consecutive launches over
// batch chunks (the backward's per-batch item prefix lives in LDS).
fa_status_t run_backward(const fa_bwd_params* p, int kind, void* stream_v) {
    fa_status_t st = validate_bwd(p, kind);
    if (st != FA_OK) return st;
    if (p->seqlen_q == 0 || (kind == FA_KIND_VARLEN && p->total_q == 0)) return FA_OK;
    const bool var = kind == FA_KIND_VARLEN;
    // kernel head dim (64, 128 or 256); dims above headdim read as zero
    const int kd = p->headdim <= 64 ? 64 : p->headdim <= 128 ? 128 : 256;
    for (int64_t b0 = 0; b0 < p->batch; b0 += kMaxBatch) {
        const int nb = (int)std::min<int64_t>(kMaxBatch, p->batch - b0);
        // dense tensors move to batch entry b0; varlen rows are addressed by
        // the (absolute) cu_seqlens prefix values
        auto bt = [&](auto* ptr, int64_t stride) { return var ? ptr : boff(ptr, b0, stride, 2); };
        fa::BwdArgs a{};
        a.q = bt(p->q, p->q_batch_stride);
        a.q_sb = p->q_batch_stride;
        a.q_si = p->q_row_stride;
        a.q_sh = p->q_head_stride;
        a.k = bt(p->k, p->k_batch_stride);
        a.k_sb = p->k_batch_stride;
        a.k_si = p->k_row_stride;
        a.k_sh = p->k_head_stride;
        a.v = bt(p->v, p->v_batch_stride);
        a.v_sb = p->v_batch_stride;
        a.v_si = p->v_row_stride;
        a.v_sh = p->v_head_stride;
        a.out = bt(p->out, p->out_batch_stride);
        a.o_sb = p->out_batch_stride;
        a.o_si = p->out_row_stride;
        a.o_sh = p->out_head_stride;
        a.dout = bt(p->dout, p->dout_batch_stride);
        a.do_sb = p->dout_batch_stride;
        a.do_si = p->dout_row_stride;
        a.do_sh = p->dout_head_stride;
        a.dq = bt(p->dq, p->dq_batch_stride);
        a.dq_sb = p->dq_batch_stride;
        a.dq_si = p->dq_row_stride;
        a.dq_sh = p->dq_head_stride;
        a.dk = bt(p->dk, p->dk_batch_stride);
        a.dk_sb = p->dk_batch_stride;
        a.dk_si = p->dk_row_stride;
        a.dk_sh = p->dk_head_stride;
        a.dv = bt(p->dv, p->dv_batch_stride);
        a.dv_sb = p->dv_batch_stride;
        a.dv_si = p->dv_row_stride;
        a.dv_sh = p->dv_head_stride;
        if (var) {
            a.lse_sb = 0;
            a.lse_sh = p->total_q;
            a.lse = p->softmax_lse;
            a.dsum = p->softmax_d;
        } else {
            a.lse_sb = (int64_t)p->nheads * p->seqlen_q;
            a.lse_sh = p->seqlen_q;
            a.lse = p->softmax_lse + (int64_t)b0 * a.lse_sb;
            a.dsum = p->softmax_d + (int64_t)b0 * a.lse_sb;
        }
        a.cu_seqlens_q = var ? p->cu_seqlens_q + b0 : nullptr;
        a.cu_seqlens_k = var ? p->cu_seqlens_k + b0 : nullptr;
        a.alibi = p->alibi_slopes ? p->alibi_slopes + (int64_t)b0 * p->alibi_batch_stride : nullptr;
        a.alibi_sb = p->alibi_batch_stride;
        a.scale = p->softmax_scale;
        a.scale_log2 = p->softmax_scale * 1.4426950408889634f;
        a.softcap = p->softcap;
        a.B = nb;
        a.Sq = p->seqlen_q;
        a.Sk = p->seqlen_k;
        a.H = p->nheads;
        a.Hk = p->nheads_k;
        a.g = p->nheads / p->nheads_k;
        a.hd = p->headdim;
        a.total_q = p->total_q;
        // window normalisation as in the forward (flash_api.cpp:483-494)
        int wl = p->window_size_left < 0 ? -1 : p->window_size_left;
        int wr = p->window_size_right < 0 ? -1 : p->window_size_right;
        if (p->is_causal) wr = 0;
        a.wl = wl;
        a.wr = wr;
        a.chunk = p->attention_chunk;
        const int64_t gkv = (int64_t)nb * p->nheads_k * (((int64_t)p->seqlen_k + fa::bwd_key_block(kd) - 1) / fa::bwd_key_block(kd));
        const int64_t gq = (int64_t)nb * p->nheads_k *
                           (((int64_t)p->seqlen_q * a.g + fa::bwd_row_block(kd) - 1) / fa::bwd_row_block(kd));
        // the kernels walk their work items in alternating passes over the
        // grid: same-length sequences run on one workgroup per CU taking
        // several items each (B4 S4096 H32/8 causal the same as with 2 x CUs
        // workgroups, B2 3-4 % faster), ragged ones on one workgroup per item
        // (up to 16 x CUs)
        const int cap = (p->cu_seqlens_q ? 16 : 1) * cu_count();
        const int grid_kv = (int)std::max<int64_t>(1, std::min<int64_t>(gkv, cap));
        const int grid_q = (int)std::max<int64_t>(1, std::min<int64_t>(gq, cap));
        hipError_t e = fa::launch_bwd(a, p->dtype, kd, grid_kv, grid_q, static_cast<hipStream_t>(stream_v));
        if (e != hipSuccess) return fail(FA_EHIP, "backward launch failed: %s", hipGetErrorString(e));
    }
    return FA_OK;
}

}  // namespace

namespace fa {
// For the no-allocation entry point (fa_noalloc.hip): the kvcache forward on
// a scratch buffer the library owns, and its error reporting.
fa_status_t forward_kvcache_on(const fa_fwd_params* p, void* stream, void* scratch, size_t bytes) {
    return run_forward_ws(p, FA_KIND_KVCACHE, stream, scratch, bytes);
}
fa_status_t report_error(fa_status_t st, const char* msg) { return fail(st, "%s", msg); }
}  // namespace fa

extern "C" {

int fa_abi_version(void) { return FA_MI355X_ABI_VERSION; }

const char* fa_last_error(void) { return g_err.c_str(); }

fa_status_t fa_validate(const fa_fwd_params* p, int32_t kind) { return validate(p, kind); }

fa_status_t fa_fwd_workspace_size(const fa_fwd_params* p, int32_t kind, size_t* bytes) {
    if (!bytes) return fail(FA_EINVAL, "bytes must not be null");
    fa_status_t st = validate(p, kind);
    if (st != FA_OK) return st;
    Plan pl;
    make_plan(p, kind, pl);
    *bytes = pl.total;
    return FA_OK;
}

fa_status_t fa_mha_fwd_kvcache(const fa_fwd_params* p, void* stream) { return run_forward(p, FA_KIND_KVCACHE, stream); }

fa_status_t fa_mha_fwd(const fa_fwd_params* p, void* stream) { return run_forward(p, FA_KIND_DENSE, stream); }

fa_status_t fa_mha_varlen_fwd(const fa_fwd_params* p, void* stream) { return run_forward(p, FA_KIND_VARLEN, stream); }

fa_status_t fa_combine(const float* out_partial, const float* lse_partial, int32_t num_splits, int64_t rows,
                       int32_t headdim_v, void* out, int64_t out_row_stride, int32_t out_dtype, float* lse,
                       void* stream) {
    if (!out_partial || !lse_partial || !out) return fail(FA_EINVAL, "out_partial, lse_partial and out are required");
    if (num_splits < 1 || rows < 0) return fail(FA_EINVAL, "num_splits must be >= 1 and rows >= 0");
    if (headdim_v < 4 || headdim_v % 4) return fail(FA_EINVAL, "headdim_v must be a positive multiple of 4");
    if (out_dtype != FA_DTYPE_FP16 && out_dtype != FA_DTYPE_BF16 && out_dtype != FA_DTYPE_FP32)
        return fail(FA_EINVAL, "out_dtype must be fp16, bf16 or fp32");
    if (out_row_stride < headdim_v || out_row_stride % 4)
        return fail(FA_EINVAL, "out_row_stride must be >= headdim_v and a multiple of 4");
    if (!aligned16(out_partial) || !aligned16(out)) return fail(FA_EINVAL, "out_partial and out must be 16-byte aligned");
    if (rows == 0) return FA_OK;
    hipError_t e = fa::launch_combine_flat(out_partial, lse_partial, num_splits, rows, headdim_v, out, out_row_stride,
                                           out_dtype, lse, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(FA_EHIP, "combine launch failed: %s", hipGetErrorString(e));
    return FA_OK;
}

fa_status_t fa_validate_bwd(const fa_bwd_params* p, int32_t kind) { return validate_bwd(p, kind); }

fa_status_t fa_bwd_workspace_size(const fa_bwd_params* p, int32_t kind, size_t* bytes) {
    if (!bytes) return fail(FA_EINVAL, "bytes must not be null");
    fa_status_t st = validate_bwd(p, kind);
    if (st != FA_OK) return st;
    *bytes = 0;
    return FA_OK;
}

fa_status_t fa_mha_bwd(const fa_bwd_params* p, void* stream) { return run_backward(p, FA_KIND_DENSE, stream); }

fa_status_t fa_mha_varlen_bwd(const fa_bwd_params* p, void* stream) { return run_backward(p, FA_KIND_VARLEN, stream); }

}  // extern "C"
