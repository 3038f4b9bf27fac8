// fa_torch_ops.cpp -- PyTorch-ROCm operators over the C ABI (libfa_mi355x.so).
//
// Registers torch.ops.fa_mi355x.{fwd_kvcache, fwd_kvcache_v3, fwd, varlen_fwd, fwd_combine,
// fwd_combine_out, bwd, varlen_bwd}.
// Argument order and meaning follow the reference pybind entry points
// (csrc/arch22/flash_attn_npu_v2/flash_api.cpp: mha_fwd_kvcache :356-377,
// mha_fwd :628-640, mha_varlen_fwd :828-850, bound at :1301-1309). Unlike the
// reference op (flash_attn_npu_v3/interface_arch22.py:63, mutates_args=()),
// the kvcache op declares that it writes k_cache / v_cache.
//
// This layer only converts tensors to fa_fwd_params, allocates outputs and
// the workspace from the caching allocator, and picks the current HIP stream.
// Errors from the library surface as RuntimeError with the library's message.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <cmath>
#include <optional>

#include "../../../include/fa_mi355x.h"

namespace {

using at::Tensor;
using OptT = std::optional<Tensor>;

int32_t dtype_code(const Tensor& t) {
    if (t.scalar_type() == at::kHalf) return FA_DTYPE_FP16;
    if (t.scalar_type() == at::kBFloat16) return FA_DTYPE_BF16;
    if (t.scalar_type() == at::kFloat8_e4m3fn) return FA_DTYPE_FP8_E4M3;
    TORCH_CHECK(false, "FlashAttention only support fp16 and bf16 data type");
}

// out has q's shape; FP8 (e4m3) inputs give a bf16 out, as in Dao's v3 API
at::TensorOptions out_options(const Tensor& q) {
    return q.scalar_type() == at::kFloat8_e4m3fn ? q.options().dtype(at::kBFloat16) : q.options();
}

void check_status(fa_status_t st) { TORCH_CHECK(st == FA_OK, "fa_mi355x: ", fa_last_error()); }

void check_dev(const Tensor& t, const Tensor& q, const char* name) {
    TORCH_CHECK(t.is_cuda(), name, " must be on a GPU device");
    TORCH_CHECK(t.device() == q.device(), name, " must be on the same device as q");
}

const int32_t* i32_ptr(const OptT& t, const Tensor& q, const char* name) {
    if (!t.has_value()) return nullptr;
    check_dev(*t, q, name);
    TORCH_CHECK(t->scalar_type() == at::kInt, name, " must have dtype int32");
    TORCH_CHECK(t->stride(-1) == 1, name, " must have contiguous last dimension");
    return t->data_ptr<int32_t>();
}

Tensor workspace_for(const fa_fwd_params& p, int32_t kind, const Tensor& q) {
    size_t bytes = 0;
    check_status(fa_fwd_workspace_size(&p, kind, &bytes));
    return at::empty({(int64_t)std::max<size_t>(bytes, 256)}, q.options().dtype(at::kByte));
}

// The workspace of a call: the caller's (the region of a v3 scheduler_metadata
// buffer after its header), checked against what the plan needs, or a fresh
// one from the caching allocator. Sets p.workspace / p.workspace_bytes.
Tensor attach_workspace(fa_fwd_params& p, int32_t kind, const Tensor& q, const OptT& given) {
    Tensor ws;
    if (given.has_value()) {
        ws = *given;
        size_t bytes = 0;
        check_status(fa_fwd_workspace_size(&p, kind, &bytes));
        TORCH_CHECK(ws.scalar_type() == at::kByte && ws.is_contiguous(), "scheduler_metadata must be a contiguous uint8 tensor");
        TORCH_CHECK(ws.device() == q.device(), "scheduler_metadata must be on the device of q");
        TORCH_CHECK((size_t)ws.numel() >= bytes, "scheduler_metadata was made for a different call: this call needs ",
                    bytes, " bytes of workspace, the metadata holds ", ws.numel());
    } else {
        ws = workspace_for(p, kind, q);
    }
    p.workspace = ws.data_ptr();
    p.workspace_bytes = (size_t)ws.numel();
    return ws;
}

void* cur_stream() { return (void*)c10::hip::getCurrentHIPStream().stream(); }

void set_window(fa_fwd_params& p, bool is_causal, int64_t wl, int64_t wr) {
    p.is_causal = is_causal ? 1 : 0;
    p.window_size_left = (int32_t)wl;
    p.window_size_right = (int32_t)wr;
}

// q_descale / k_descale / v_descale: fp32 (batch_size, num_heads_k), read for FP8 inputs only
// (their shape per csrc/arch22/flash_attn_npu_v3/flash_api.cpp:82-84 of the reference)
void set_descale(fa_fwd_params& p, const OptT& qd, const OptT& kd, const OptT& vd, const Tensor& q, int64_t batch) {
    auto one = [&](const OptT& t, const char* name, const float*& ptr, int64_t& sb, int64_t& sh) {
        if (!t.has_value()) return;
        check_dev(*t, q, name);
        TORCH_CHECK(t->scalar_type() == at::kFloat, name, " must have dtype fp32");
        TORCH_CHECK(t->dim() == 2 && t->size(0) == batch && t->size(1) == p.nheads_k, name,
                    " must have shape (batch_size, num_heads_k)");
        ptr = t->data_ptr<float>();
        sb = t->stride(0);
        sh = t->stride(1);
    };
    one(qd, "q_descale", p.q_descale, p.q_descale_batch_stride, p.q_descale_head_stride);
    one(kd, "k_descale", p.k_descale, p.k_descale_batch_stride, p.k_descale_head_stride);
    one(vd, "v_descale", p.v_descale, p.v_descale_batch_stride, p.v_descale_head_stride);
}

void set_alibi(fa_fwd_params& p, const OptT& alibi, const Tensor& q, int64_t batch, int64_t nheads) {
    if (!alibi.has_value()) return;
    check_dev(*alibi, q, "alibi_slopes");
    TORCH_CHECK(alibi->scalar_type() == at::kFloat, "ALiBi slopes must have dtype fp32");
    TORCH_CHECK(alibi->stride(-1) == 1, "ALiBi slopes tensor must have contiguous last dimension");
    TORCH_CHECK(alibi->sizes() == at::IntArrayRef({nheads}) || alibi->sizes() == at::IntArrayRef({batch, nheads}),
                "alibi_slopes must have shape (nheads) or (batch_size, nheads)");
    p.alibi_slopes = alibi->data_ptr<float>();
    p.alibi_batch_stride = alibi->dim() == 2 ? alibi->stride(0) : 0;
}

// ---- flash_attn_with_kvcache -----------------------------------------------------------
// Shared by the v2 op (the reference's fwd_kvcache argument order) and the v3
// op, which adds ragged queries / new tokens, rotary positions and
// attention_chunk. q is (B, Sq, H, D), or (total_q, H, D) with cu_seqlens_q;
// k / v are (B, S_new, Hk, D), or (total_k_new, Hk, D) with cu_seqlens_k_new.
std::tuple<Tensor, Tensor> kvcache_impl(const Tensor& q, Tensor& kcache, Tensor& vcache, const OptT& k_new,
                                        const OptT& v_new, const OptT& seqlens_k, const OptT& rotary_cos,
                                        const OptT& rotary_sin, const OptT& cache_batch_idx, const OptT& leftpad_k,
                                        const OptT& block_table, const OptT& alibi_slopes, const OptT& cu_seqlens_q,
                                        const OptT& cu_seqlens_k_new, int64_t max_seqlen_q,
                                        const OptT& rotary_seqlens, double softmax_scale, bool is_causal,
                                        int64_t window_size_left, int64_t window_size_right, int64_t attention_chunk,
                                        double softcap, bool is_rotary_interleaved, int64_t num_splits,
                                        const OptT& q_descale, const OptT& k_descale, const OptT& v_descale,
                                        const OptT& workspace, const OptT& qv, std::optional<bool> pack_gqa) {
    c10::DeviceGuard guard(q.device());
    TORCH_CHECK(q.is_cuda(), "q must be on a GPU device");
    check_dev(kcache, q, "k_cache");
    check_dev(vcache, q, "v_cache");
    const int32_t dt = dtype_code(q);
    TORCH_CHECK(kcache.scalar_type() == q.scalar_type() && vcache.scalar_type() == q.scalar_type(),
                "query and key/value must have the same dtype");
    const bool ragged_q = cu_seqlens_q.has_value();
    if (ragged_q) {
        TORCH_CHECK(q.dim() == 3, "q must have shape (total_q, num_heads, head_size) with cu_seqlens_q");
    } else {
        TORCH_CHECK(q.dim() == 4, "q must have shape (batch_size, seqlen_q, num_heads, head_size)");
    }
    TORCH_CHECK(kcache.dim() == 4 && vcache.dim() == 4, "k_cache/v_cache must be 4-dimensional");
    TORCH_CHECK(q.stride(-1) == 1 && kcache.stride(-1) == 1 && vcache.stride(-1) == 1,
                "Input tensor must have contiguous last dimension");
    const bool paged = block_table.has_value();
    const int64_t batch = ragged_q ? cu_seqlens_q->numel() - 1 : q.size(0);
    TORCH_CHECK(batch >= 1, "batch size must be positive");
    fa_fwd_params p{};
    p.abi_version = FA_MI355X_ABI_VERSION;
    p.dtype = dt;
    p.batch = (int32_t)batch;
    p.nheads = (int32_t)q.size(-2);
    p.headdim = (int32_t)q.size(-1);
    p.nheads_k = (int32_t)kcache.size(2);
    p.headdim_v = (int32_t)vcache.size(3);
    TORCH_CHECK(kcache.size(3) == p.headdim, "k_cache head size must match q");
    TORCH_CHECK(vcache.sizes() == kcache.sizes(), "v_cache must have the same shape as k_cache");
    p.batch_cache = (int32_t)kcache.size(0);
    p.seqlen_k = (int32_t)kcache.size(1);
    p.q = q.data_ptr();
    if (ragged_q) {
        p.cu_seqlens_q = i32_ptr(cu_seqlens_q, q, "cu_seqlens_q");
        p.seqlen_q = (int32_t)max_seqlen_q;
        p.total_q = (int32_t)q.size(0);
        p.q_batch_stride = 0;
        p.q_row_stride = q.stride(0);
        p.q_head_stride = q.stride(1);
    } else {
        p.seqlen_q = (int32_t)q.size(1);
        p.q_batch_stride = q.stride(0);
        p.q_row_stride = q.stride(1);
        p.q_head_stride = q.stride(2);
    }
    p.k = kcache.data_ptr();
    p.k_batch_stride = kcache.stride(0);
    p.k_row_stride = kcache.stride(1);
    p.k_head_stride = kcache.stride(2);
    p.v = vcache.data_ptr();
    p.v_batch_stride = vcache.stride(0);
    p.v_row_stride = vcache.stride(1);
    p.v_head_stride = vcache.stride(2);
    if (paged) {
        p.block_table = i32_ptr(block_table, q, "block_table");
        TORCH_CHECK(block_table->dim() == 2, "block_table must be 2-dimensional");
        p.block_table_batch_stride = block_table->stride(0);
        p.max_blocks_per_seq = (int32_t)block_table->size(1);
        p.block_table_rows = (int32_t)block_table->size(0);
        p.page_block_size = (int32_t)kcache.size(1);
        const int64_t rows_needed = cache_batch_idx.has_value() ? 1 : batch;
        TORCH_CHECK(block_table->size(0) >= rows_needed, "block_table must have a row per batch entry");
    }
    Tensor kn, vn;
    if (k_new.has_value()) {
        TORCH_CHECK(v_new.has_value(), "If key is supplied, value must also be passed in");
        TORCH_CHECK(seqlens_k.has_value(), "If key is supplied, seqlens_k must also be passed in");
        kn = k_new->stride(-1) == 1 ? *k_new : k_new->contiguous();
        vn = v_new->stride(-1) == 1 ? *v_new : v_new->contiguous();
        check_dev(kn, q, "k");
        check_dev(vn, q, "v");
        TORCH_CHECK(kn.scalar_type() == q.scalar_type() && vn.scalar_type() == q.scalar_type(),
                    "Key and value must have the same dtype as query");
        TORCH_CHECK(vn.sizes() == kn.sizes(), "v must have the same shape as k");
        p.k_new = kn.data_ptr();
        p.v_new = vn.data_ptr();
        if (cu_seqlens_k_new.has_value()) {
            TORCH_CHECK(kn.dim() == 3 && kn.size(1) == p.nheads_k && kn.size(2) == p.headdim,
                        "k must have shape (total_k_new, num_heads_k, head_size) with cu_seqlens_k_new");
            TORCH_CHECK(cu_seqlens_k_new->numel() == batch + 1, "cu_seqlens_k_new must have shape (batch_size + 1)");
            p.cu_seqlens_k_new = i32_ptr(cu_seqlens_k_new, q, "cu_seqlens_k_new");
            p.total_k_new = (int32_t)kn.size(0);
            p.knew_row_stride = kn.stride(0);
            p.knew_head_stride = kn.stride(1);
            p.vnew_row_stride = vn.stride(0);
            p.vnew_head_stride = vn.stride(1);
        } else {
            TORCH_CHECK(kn.dim() == 4 && kn.size(0) == batch && kn.size(2) == p.nheads_k && kn.size(3) == p.headdim,
                        "k must have shape (batch_size, seqlen_new, num_heads_k, head_size)");
            p.knew_batch_stride = kn.stride(0);
            p.knew_row_stride = kn.stride(1);
            p.knew_head_stride = kn.stride(2);
            p.vnew_batch_stride = vn.stride(0);
            p.vnew_row_stride = vn.stride(1);
            p.vnew_head_stride = vn.stride(2);
            p.seqlen_new = (int32_t)kn.size(1);
        }
    } else {
        TORCH_CHECK(!v_new.has_value(), "If value is supplied, key must also be passed in");
        TORCH_CHECK(!cu_seqlens_k_new.has_value(), "cu_seqlens_k_new is given without new keys k / v");
    }
    auto per_batch = [&](const OptT& t, const char* name) -> const int32_t* {
        if (!t.has_value()) return nullptr;
        TORCH_CHECK(t->numel() == batch, name, " must have shape (batch_size)");
        return i32_ptr(t, q, name);
    };
    p.cache_seqlens = per_batch(seqlens_k, "seqlens_k");
    p.cache_batch_idx = per_batch(cache_batch_idx, "cache_batch_idx");
    p.cache_leftpad = per_batch(leftpad_k, "cache_leftpad");
    p.rotary_seqlens = per_batch(rotary_seqlens, "rotary_seqlens");
    if (leftpad_k.has_value()) {
        TORCH_CHECK(seqlens_k.has_value(), "cache_leftpad needs cache_seqlens");
    }
    if (rotary_cos.has_value()) {
        TORCH_CHECK(rotary_sin.has_value(), "rotary_sin must be given with rotary_cos");
        check_dev(*rotary_cos, q, "rotary_cos");
        check_dev(*rotary_sin, q, "rotary_sin");
        TORCH_CHECK(rotary_cos->scalar_type() == q.scalar_type() && rotary_sin->scalar_type() == q.scalar_type(),
                    "rotary_cos/sin must have the same dtype as query");
        TORCH_CHECK(rotary_cos->dim() == 2 && rotary_cos->sizes() == rotary_sin->sizes(),
                    "rotary_cos/sin must have shape (seqlen_ro, rotary_dim / 2)");
        TORCH_CHECK(rotary_cos->is_contiguous() && rotary_sin->is_contiguous(), "rotary_cos/sin must be contiguous");
        p.rotary_cos = rotary_cos->data_ptr();
        p.rotary_sin = rotary_sin->data_ptr();
        p.rotary_dim = (int32_t)rotary_cos->size(1) * 2;
        p.seqlen_ro = (int32_t)rotary_cos->size(0);
        p.rotary_interleaved = is_rotary_interleaved ? 1 : 0;
    }
    set_alibi(p, alibi_slopes, q, batch, p.nheads);
    p.softmax_scale = (float)softmax_scale;
    p.softcap = (float)softcap;
    set_window(p, is_causal, window_size_left, window_size_right);
    p.attention_chunk = (int32_t)attention_chunk;
    p.num_splits = (int32_t)num_splits;
    set_descale(p, q_descale, k_descale, v_descale, q, batch);
    Tensor qvc;
    if (qv.has_value()) {
        check_dev(*qv, q, "qv");
        TORCH_CHECK(qv->scalar_type() == q.scalar_type(), "qv must have the same dtype as query");
        TORCH_CHECK(qv->dim() == q.dim() && qv->size(0) == q.size(0) && qv->size(-2) == q.size(-2) &&
                        (ragged_q || qv->size(1) == q.size(1)) && qv->size(-1) == p.headdim_v,
                    "qv must have shape (batch_size, seqlen_q, num_heads, head_size_v), or (total_q, num_heads, "
                    "head_size_v) with cu_seqlens_q");
        qvc = qv->stride(-1) == 1 ? *qv : qv->contiguous();
        p.qv = qvc.data_ptr();
        if (ragged_q) {
            p.qv_row_stride = qvc.stride(0);
            p.qv_head_stride = qvc.stride(1);
        } else {
            p.qv_batch_stride = qvc.stride(0);
            p.qv_row_stride = qvc.stride(1);
            p.qv_head_stride = qvc.stride(2);
        }
    }
    p.no_pack_gqa = pack_gqa.has_value() && !*pack_gqa ? 1 : 0;
    Tensor out = at::empty(q.sizes(), out_options(q));
    Tensor lse = ragged_q ? at::empty({q.size(1), q.size(0)}, q.options().dtype(at::kFloat))
                          : at::empty({q.size(0), q.size(2), q.size(1)}, q.options().dtype(at::kFloat));
    p.out = out.data_ptr();
    if (ragged_q) {
        p.out_batch_stride = 0;
        p.out_row_stride = out.stride(0);
        p.out_head_stride = out.stride(1);
    } else {
        p.out_batch_stride = out.stride(0);
        p.out_row_stride = out.stride(1);
        p.out_head_stride = out.stride(2);
    }
    p.softmax_lse = lse.data_ptr<float>();
    Tensor ws = attach_workspace(p, FA_KIND_KVCACHE, q, workspace);
    check_status(fa_mha_fwd_kvcache(&p, cur_stream()));
    return {out, lse};
}

std::tuple<Tensor, Tensor> fwd_kvcache(const Tensor& q, Tensor& kcache, Tensor& vcache, const OptT& k_new,
                                       const OptT& v_new, const OptT& seqlens_k, const OptT& rotary_cos,
                                       const OptT& rotary_sin, const OptT& cache_batch_idx, const OptT& leftpad_k,
                                       const OptT& block_table, const OptT& alibi_slopes, double softmax_scale,
                                       bool is_causal, int64_t window_size_left, int64_t window_size_right,
                                       double softcap, bool is_rotary_interleaved, int64_t num_splits) {
    return kvcache_impl(q, kcache, vcache, k_new, v_new, seqlens_k, rotary_cos, rotary_sin, cache_batch_idx,
                        leftpad_k, block_table, alibi_slopes, std::nullopt, std::nullopt, 0, std::nullopt,
                        softmax_scale, is_causal, window_size_left, window_size_right, 0, softcap,
                        is_rotary_interleaved, num_splits, std::nullopt, std::nullopt, std::nullopt, std::nullopt,
                        std::nullopt, std::nullopt);
}

std::tuple<Tensor, Tensor> fwd_kvcache_v3(const Tensor& q, Tensor& kcache, Tensor& vcache, const OptT& k_new,
                                          const OptT& v_new, const OptT& seqlens_k, const OptT& rotary_cos,
                                          const OptT& rotary_sin, const OptT& cache_batch_idx,
                                          const OptT& leftpad_k, const OptT& block_table,
                                          const OptT& alibi_slopes, const OptT& cu_seqlens_q,
                                          const OptT& cu_seqlens_k_new, int64_t max_seqlen_q,
                                          const OptT& rotary_seqlens, double softmax_scale, bool is_causal,
                                          int64_t window_size_left, int64_t window_size_right,
                                          int64_t attention_chunk, double softcap, bool is_rotary_interleaved,
                                          int64_t num_splits, const OptT& q_descale, const OptT& k_descale,
                                          const OptT& v_descale, const OptT& workspace, const OptT& qv,
                                          std::optional<bool> pack_gqa) {
    return kvcache_impl(q, kcache, vcache, k_new, v_new, seqlens_k, rotary_cos, rotary_sin, cache_batch_idx,
                        leftpad_k, block_table, alibi_slopes, cu_seqlens_q, cu_seqlens_k_new, max_seqlen_q,
                        rotary_seqlens, softmax_scale, is_causal, window_size_left, window_size_right,
                        attention_chunk, softcap, is_rotary_interleaved, num_splits, q_descale, k_descale,
                        v_descale, workspace, qv, pack_gqa);
}

// ---- flash_attn_func ------------------------------------------------------------------------
std::tuple<Tensor, Tensor> fwd(const Tensor& q, const Tensor& k, const Tensor& v, const OptT& alibi_slopes,
                               double p_dropout, double softmax_scale, bool is_causal, int64_t window_size_left,
                               int64_t window_size_right, double softcap, int64_t attention_chunk,
                               const OptT& q_descale, const OptT& k_descale, const OptT& v_descale,
                               int64_t num_splits, const OptT& workspace, std::optional<bool> pack_gqa) {
    c10::DeviceGuard guard(q.device());
    TORCH_CHECK(q.is_cuda(), "q must be on a GPU device");
    check_dev(k, q, "k");
    check_dev(v, q, "v");
    const int32_t dt = dtype_code(q);
    TORCH_CHECK(k.scalar_type() == q.scalar_type() && v.scalar_type() == q.scalar_type(),
                "query and key/value must have the same dtype");
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "q, k, v must be 4-dimensional (batch, seqlen, heads, dim)");
    TORCH_CHECK(q.stride(-1) == 1 && k.stride(-1) == 1 && v.stride(-1) == 1,
                "Input tensor must have contiguous last dimension");
    TORCH_CHECK(k.size(0) == q.size(0) && v.sizes() == k.sizes(), "k and v must have shape (batch_size, seqlen_k, num_heads_k, head_size)");
    TORCH_CHECK(k.size(3) == q.size(3), "k head size must match q");
    fa_fwd_params p{};
    p.abi_version = FA_MI355X_ABI_VERSION;
    p.dtype = dt;
    p.batch = (int32_t)q.size(0);
    p.seqlen_q = (int32_t)q.size(1);
    p.nheads = (int32_t)q.size(2);
    p.headdim = (int32_t)q.size(3);
    p.nheads_k = (int32_t)k.size(2);
    p.headdim_v = (int32_t)v.size(3);
    p.seqlen_k = (int32_t)k.size(1);
    p.batch_cache = p.batch;
    p.q = q.data_ptr();
    p.q_batch_stride = q.stride(0);
    p.q_row_stride = q.stride(1);
    p.q_head_stride = q.stride(2);
    p.k = const_cast<void*>(k.data_ptr());
    p.k_batch_stride = k.stride(0);
    p.k_row_stride = k.stride(1);
    p.k_head_stride = k.stride(2);
    p.v = const_cast<void*>(v.data_ptr());
    p.v_batch_stride = v.stride(0);
    p.v_row_stride = v.stride(1);
    p.v_head_stride = v.stride(2);
    set_alibi(p, alibi_slopes, q, q.size(0), q.size(2));
    p.dropout_p = (float)p_dropout;
    p.softmax_scale = (float)softmax_scale;
    p.softcap = (float)softcap;
    set_window(p, is_causal, window_size_left, window_size_right);
    p.attention_chunk = (int32_t)attention_chunk;
    TORCH_CHECK(num_splits >= 0, "num_splits must be >= 0");
    p.num_splits = (int32_t)num_splits;
    set_descale(p, q_descale, k_descale, v_descale, q, q.size(0));
    Tensor out = at::empty(q.sizes(), out_options(q));
    Tensor lse = at::empty({q.size(0), q.size(2), q.size(1)}, q.options().dtype(at::kFloat));
    p.out = out.data_ptr();
    p.out_batch_stride = out.stride(0);
    p.out_row_stride = out.stride(1);
    p.out_head_stride = out.stride(2);
    p.softmax_lse = lse.data_ptr<float>();
    p.no_pack_gqa = pack_gqa.has_value() && !*pack_gqa ? 1 : 0;
    Tensor ws = attach_workspace(p, FA_KIND_DENSE, q, workspace);
    check_status(fa_mha_fwd(&p, cur_stream()));
    return {out, lse};
}

// ---- flash_attn_varlen_func -----------------------------------------------------------------------
std::tuple<Tensor, Tensor> varlen_fwd(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& cu_seqlens_q,
                                      const OptT& cu_seqlens_k, const OptT& seqused_k, const OptT& block_table,
                                      const OptT& alibi_slopes,
                                      int64_t max_seqlen_q, int64_t max_seqlen_k, double p_dropout,
                                      double softmax_scale, bool is_causal, int64_t window_size_left,
                                      int64_t window_size_right, double softcap, int64_t attention_chunk,
                                      const OptT& q_descale, const OptT& k_descale, const OptT& v_descale,
                                      int64_t num_splits, const OptT& workspace, std::optional<bool> pack_gqa) {
    c10::DeviceGuard guard(q.device());
    TORCH_CHECK(q.is_cuda(), "q must be on a GPU device");
    check_dev(k, q, "k");
    check_dev(v, q, "v");
    const int32_t dt = dtype_code(q);
    TORCH_CHECK(k.scalar_type() == q.scalar_type() && v.scalar_type() == q.scalar_type(),
                "query and key/value must have the same dtype");
    TORCH_CHECK(q.dim() == 3, "q must have shape (total_q, num_heads, head_size)");
    TORCH_CHECK(q.stride(-1) == 1 && k.stride(-1) == 1 && v.stride(-1) == 1,
                "Input tensor must have contiguous last dimension");
    const bool paged = block_table.has_value();
    fa_fwd_params p{};
    p.abi_version = FA_MI355X_ABI_VERSION;
    p.dtype = dt;
    p.batch = (int32_t)(cu_seqlens_q.numel() - 1);
    TORCH_CHECK(!cu_seqlens_k.has_value() || cu_seqlens_k->numel() == cu_seqlens_q.numel(),
                "cu_seqlens_q and cu_seqlens_k must have the same length");
    TORCH_CHECK(!seqused_k.has_value() || seqused_k->numel() == p.batch, "seqused_k must have shape (batch_size)");
    p.seqlen_q = (int32_t)max_seqlen_q;
    p.total_q = (int32_t)q.size(0);
    p.nheads = (int32_t)q.size(1);
    p.headdim = (int32_t)q.size(2);
    p.q = q.data_ptr();
    p.q_batch_stride = 0;
    p.q_row_stride = q.stride(0);
    p.q_head_stride = q.stride(1);
    if (paged) {
        TORCH_CHECK(k.dim() == 4, "paged k must have shape (num_blocks, page_block_size, num_heads_k, head_size)");
        p.nheads_k = (int32_t)k.size(2);
        p.headdim_v = (int32_t)v.size(3);
        p.k_batch_stride = k.stride(0);
        p.k_row_stride = k.stride(1);
        p.k_head_stride = k.stride(2);
        p.v_batch_stride = v.stride(0);
        p.v_row_stride = v.stride(1);
        p.v_head_stride = v.stride(2);
        p.block_table = i32_ptr(block_table, q, "block_table");
        p.block_table_batch_stride = block_table->stride(0);
        p.max_blocks_per_seq = (int32_t)block_table->size(1);
        p.block_table_rows = (int32_t)block_table->size(0);
        p.page_block_size = (int32_t)k.size(1);
        p.batch_cache = (int32_t)k.size(0);
    } else {
        TORCH_CHECK(k.dim() == 3, "k must have shape (total_k, num_heads_k, head_size)");
        p.nheads_k = (int32_t)k.size(1);
        p.headdim_v = (int32_t)v.size(2);
        p.k_batch_stride = 0;
        p.k_row_stride = k.stride(0);
        p.k_head_stride = k.stride(1);
        p.v_batch_stride = 0;
        p.v_row_stride = v.stride(0);
        p.v_head_stride = v.stride(1);
        p.batch_cache = p.batch;
    }
    p.seqlen_k = (int32_t)max_seqlen_k;
    p.k = const_cast<void*>(k.data_ptr());
    p.v = const_cast<void*>(v.data_ptr());
    p.cu_seqlens_q = i32_ptr(cu_seqlens_q, q, "cu_seqlens_q");
    p.cu_seqlens_k = i32_ptr(cu_seqlens_k, q, "cu_seqlens_k");
    p.cache_seqlens = i32_ptr(seqused_k, q, "seqused_k");
    set_alibi(p, alibi_slopes, q, p.batch, q.size(1));
    p.dropout_p = (float)p_dropout;
    p.softmax_scale = (float)softmax_scale;
    p.softcap = (float)softcap;
    set_window(p, is_causal, window_size_left, window_size_right);
    p.attention_chunk = (int32_t)attention_chunk;
    TORCH_CHECK(num_splits >= 0, "num_splits must be >= 0");
    p.num_splits = (int32_t)num_splits;
    set_descale(p, q_descale, k_descale, v_descale, q, p.batch);
    Tensor out = at::empty(q.sizes(), out_options(q));
    Tensor lse = at::empty({q.size(1), q.size(0)}, q.options().dtype(at::kFloat));
    p.out = out.data_ptr();
    p.out_batch_stride = 0;
    p.out_row_stride = out.stride(0);
    p.out_head_stride = out.stride(1);
    p.softmax_lse = lse.data_ptr<float>();
    p.no_pack_gqa = pack_gqa.has_value() && !*pack_gqa ? 1 : 0;
    Tensor ws = attach_workspace(p, FA_KIND_VARLEN, q, workspace);
    check_status(fa_mha_varlen_fwd(&p, cur_stream()));
    return {out, lse};
}

// ---- flash_attn_combine --------------------------------------------------------------------------
// combine_into writes the merged rows into `out`; fwd_combine allocates it,
// fwd_combine_out takes the caller's (declared as written by the op).
Tensor combine_into(const Tensor& out_partial, const Tensor& lse_partial, Tensor& out);

std::tuple<Tensor, Tensor> fwd_combine(const Tensor& out_partial, const Tensor& lse_partial,
                                       std::optional<at::ScalarType> out_dtype) {
    TORCH_CHECK(out_partial.dim() >= 2, "out_partial must have a split dimension and headdim_v");
    std::vector<int64_t> oshape(out_partial.sizes().begin() + 1, out_partial.sizes().end());
    Tensor out = at::empty(oshape, out_partial.options().dtype(out_dtype.has_value() ? *out_dtype : at::kFloat));
    Tensor lse = combine_into(out_partial, lse_partial, out);
    return {out, lse};
}

Tensor fwd_combine_out(const Tensor& out_partial, const Tensor& lse_partial, Tensor& out) {
    return combine_into(out_partial, lse_partial, out);
}

Tensor combine_into(const Tensor& out_partial, const Tensor& lse_partial, Tensor& out) {
    c10::DeviceGuard guard(out_partial.device());
    TORCH_CHECK(out_partial.is_cuda() && lse_partial.is_cuda(), "inputs must be on a GPU device");
    TORCH_CHECK(out_partial.scalar_type() == at::kFloat && lse_partial.scalar_type() == at::kFloat,
                "out_partial and lse_partial must be fp32");
    // out_partial (num_splits, ..., headdim_v); lse_partial (num_splits, ...)
    TORCH_CHECK(out_partial.dim() >= 2 && lse_partial.dim() == out_partial.dim() - 1,
                "lse_partial must have the shape of out_partial without its last dimension");
    for (int64_t d = 0; d < lse_partial.dim(); ++d)
        TORCH_CHECK(lse_partial.size(d) == out_partial.size(d), "lse_partial shape mismatch at dim ", d);
    Tensor po = out_partial.contiguous();
    Tensor pl = lse_partial.contiguous();
    const int64_t S = po.size(0);
    const int64_t Dv = po.size(-1);
    const int64_t R = S > 0 ? po.numel() / (S * Dv) : 0;
    TORCH_CHECK(out.device() == po.device(), "out must be on the device of out_partial");
    TORCH_CHECK(out.is_contiguous() && out.numel() == R * Dv, "out must be contiguous with ", R * Dv, " elements");
    int32_t code = out.scalar_type() == at::kFloat ? FA_DTYPE_FP32
                   : out.scalar_type() == at::kBFloat16 ? FA_DTYPE_BF16
                   : out.scalar_type() == at::kHalf ? FA_DTYPE_FP16 : -1;
    TORCH_CHECK(code >= 0, "out dtype must be fp32, bf16 or fp16");
    std::vector<int64_t> lshape(pl.sizes().begin() + 1, pl.sizes().end());
    Tensor lse = at::empty(lshape, po.options());
    check_status(fa_combine(po.data_ptr<float>(), pl.data_ptr<float>(), (int32_t)S, R, (int32_t)Dv, out.data_ptr(), Dv,
                            code, lse.data_ptr<float>(), cur_stream()));
    return lse;
}

// ---- backward (flash_attn_func / flash_attn_varlen_func autograd) ------------------------------
// The reference binds mha_bwd / mha_varlen_bwd (flash_api.cpp:1063-1299) and
// returns (dq, dk, dv, softmax_d); so does this op, which allocates dq, dk, dv.
void set_bwd_common(fa_bwd_params& p, const Tensor& dout, const Tensor& q, const Tensor& k, const Tensor& v,
                    const Tensor& out, const Tensor& lse) {
    TORCH_CHECK(q.is_cuda(), "q must be on a GPU device");
    check_dev(k, q, "k");
    check_dev(v, q, "v");
    check_dev(out, q, "out");
    check_dev(dout, q, "dout");
    check_dev(lse, q, "softmax_lse");
    p.abi_version = FA_MI355X_ABI_VERSION;
    p.dtype = dtype_code(q);
    for (const Tensor* t : {&k, &v, &out, &dout})
        TORCH_CHECK(t->scalar_type() == q.scalar_type(), "q, k, v, out and dout must have the same dtype");
    TORCH_CHECK(lse.scalar_type() == at::kFloat, "softmax_lse must be fp32");
    for (const Tensor* t : {&q, &k, &v, &out, &dout})
        TORCH_CHECK(t->stride(-1) == 1, "Input tensor must have contiguous last dimension");
}

std::tuple<Tensor, Tensor, Tensor, Tensor> bwd(const Tensor& dout, const Tensor& q, const Tensor& k, const Tensor& v,
                                               const Tensor& out, const Tensor& softmax_lse, const OptT& alibi_slopes,
                                               double p_dropout, double softmax_scale, bool is_causal,
                                               int64_t window_size_left, int64_t window_size_right, double softcap,
                                               bool deterministic, int64_t attention_chunk) {
    c10::DeviceGuard guard(q.device());
    fa_bwd_params p{};
    set_bwd_common(p, dout, q, k, v, out, softmax_lse);
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "q, k, v must have shape (batch, seqlen, heads, head_size)");
    TORCH_CHECK(dout.sizes() == q.sizes() && out.sizes() == q.sizes(), "out and dout must have the shape of q");
    TORCH_CHECK(k.sizes() == v.sizes() && k.size(0) == q.size(0) && k.size(3) == q.size(3), "k and v shapes must match q");
    const int64_t B = q.size(0), Sq = q.size(1), H = q.size(2);
    TORCH_CHECK(softmax_lse.sizes() == at::IntArrayRef({B, H, Sq}) && softmax_lse.is_contiguous(),
                "softmax_lse must be a contiguous (batch, nheads, seqlen_q) tensor");
    Tensor lse = softmax_lse;
    Tensor dq = at::empty(q.sizes(), q.options());
    Tensor dk = at::empty(k.sizes(), k.options());
    Tensor dv = at::empty(v.sizes(), v.options());
    Tensor sd = at::empty({B, H, Sq}, q.options().dtype(at::kFloat));
    p.batch = (int32_t)B;
    p.seqlen_q = (int32_t)Sq;
    p.seqlen_k = (int32_t)k.size(1);
    p.nheads = (int32_t)H;
    p.nheads_k = (int32_t)k.size(2);
    p.headdim = (int32_t)q.size(3);
    auto set4 = [](const Tensor& t, const void*& ptr, int64_t& sb, int64_t& si, int64_t& sh) {
        ptr = t.data_ptr();
        sb = t.stride(0);
        si = t.stride(1);
        sh = t.stride(2);
    };
    auto set4m = [](Tensor& t, void*& ptr, int64_t& sb, int64_t& si, int64_t& sh) {
        ptr = t.data_ptr();
        sb = t.stride(0);
        si = t.stride(1);
        sh = t.stride(2);
    };
    set4(q, p.q, p.q_batch_stride, p.q_row_stride, p.q_head_stride);
    set4(k, p.k, p.k_batch_stride, p.k_row_stride, p.k_head_stride);
    set4(v, p.v, p.v_batch_stride, p.v_row_stride, p.v_head_stride);
    set4(out, p.out, p.out_batch_stride, p.out_row_stride, p.out_head_stride);
    set4(dout, p.dout, p.dout_batch_stride, p.dout_row_stride, p.dout_head_stride);
    set4m(dq, p.dq, p.dq_batch_stride, p.dq_row_stride, p.dq_head_stride);
    set4m(dk, p.dk, p.dk_batch_stride, p.dk_row_stride, p.dk_head_stride);
    set4m(dv, p.dv, p.dv_batch_stride, p.dv_row_stride, p.dv_head_stride);
    p.softmax_lse = lse.data_ptr<float>();
    p.softmax_d = sd.data_ptr<float>();
    if (alibi_slopes.has_value()) {
        check_dev(*alibi_slopes, q, "alibi_slopes");
        TORCH_CHECK(alibi_slopes->scalar_type() == at::kFloat && alibi_slopes->stride(-1) == 1,
                    "ALiBi slopes must be fp32 with a contiguous last dimension");
        TORCH_CHECK(alibi_slopes->sizes() == at::IntArrayRef({H}) || alibi_slopes->sizes() == at::IntArrayRef({B, H}),
                    "alibi_slopes must have shape (nheads) or (batch_size, nheads)");
        p.alibi_slopes = alibi_slopes->data_ptr<float>();
        p.alibi_batch_stride = alibi_slopes->dim() == 2 ? alibi_slopes->stride(0) : 0;
    }
    p.dropout_p = (float)p_dropout;
    p.softmax_scale = (float)softmax_scale;
    p.softcap = (float)softcap;
    p.is_causal = is_causal ? 1 : 0;
    p.window_size_left = (int32_t)window_size_left;
    p.window_size_right = (int32_t)window_size_right;
    p.deterministic = deterministic ? 1 : 0;
    p.attention_chunk = (int32_t)attention_chunk;
    check_status(fa_mha_bwd(&p, cur_stream()));
    return {dq, dk, dv, sd};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> varlen_bwd(const Tensor& dout, const Tensor& q, const Tensor& k,
                                                      const Tensor& v, const Tensor& out, const Tensor& softmax_lse,
                                                      const Tensor& cu_seqlens_q, const Tensor& cu_seqlens_k,
                                                      const OptT& alibi_slopes, int64_t max_seqlen_q,
                                                      int64_t max_seqlen_k, double p_dropout, double softmax_scale,
                                                      bool is_causal, int64_t window_size_left,
                                                      int64_t window_size_right, double softcap, bool deterministic,
                                                      int64_t attention_chunk) {
    c10::DeviceGuard guard(q.device());
    fa_bwd_params p{};
    set_bwd_common(p, dout, q, k, v, out, softmax_lse);
    TORCH_CHECK(q.dim() == 3 && k.dim() == 3 && v.dim() == 3, "q, k, v must have shape (total, heads, head_size)");
    TORCH_CHECK(dout.sizes() == q.sizes() && out.sizes() == q.sizes(), "out and dout must have the shape of q");
    TORCH_CHECK(k.sizes() == v.sizes() && k.size(2) == q.size(2), "k and v shapes must match q");
    TORCH_CHECK(cu_seqlens_q.numel() == cu_seqlens_k.numel() && cu_seqlens_q.numel() >= 2,
                "cu_seqlens_q and cu_seqlens_k must have the same length >= 2");
    const int64_t T = q.size(0), H = q.size(1);
    TORCH_CHECK(softmax_lse.sizes() == at::IntArrayRef({H, T}) && softmax_lse.is_contiguous(),
                "mha_varlen_bwd: softmax_lse must be a contiguous (nheads, total_q) tensor");
    Tensor dq = at::empty(q.sizes(), q.options());
    Tensor dk = at::empty(k.sizes(), k.options());
    Tensor dv = at::empty(v.sizes(), v.options());
    Tensor sd = at::empty({H, T}, q.options().dtype(at::kFloat));
    p.batch = (int32_t)(cu_seqlens_q.numel() - 1);
    p.seqlen_q = (int32_t)max_seqlen_q;
    p.seqlen_k = (int32_t)max_seqlen_k;
    p.total_q = (int32_t)T;
    p.nheads = (int32_t)H;
    p.nheads_k = (int32_t)k.size(1);
    p.headdim = (int32_t)q.size(2);
    auto set3 = [](const Tensor& t, const void*& ptr, int64_t& sb, int64_t& si, int64_t& sh) {
        ptr = t.data_ptr();
        sb = 0;
        si = t.stride(0);
        sh = t.stride(1);
    };
    auto set3m = [](Tensor& t, void*& ptr, int64_t& sb, int64_t& si, int64_t& sh) {
        ptr = t.data_ptr();
        sb = 0;
        si = t.stride(0);
        sh = t.stride(1);
    };
    set3(q, p.q, p.q_batch_stride, p.q_row_stride, p.q_head_stride);
    set3(k, p.k, p.k_batch_stride, p.k_row_stride, p.k_head_stride);
    set3(v, p.v, p.v_batch_stride, p.v_row_stride, p.v_head_stride);
    set3(out, p.out, p.out_batch_stride, p.out_row_stride, p.out_head_stride);
    set3(dout, p.dout, p.dout_batch_stride, p.dout_row_stride, p.dout_head_stride);
    set3m(dq, p.dq, p.dq_batch_stride, p.dq_row_stride, p.dq_head_stride);
    set3m(dk, p.dk, p.dk_batch_stride, p.dk_row_stride, p.dk_head_stride);
    set3m(dv, p.dv, p.dv_batch_stride, p.dv_row_stride, p.dv_head_stride);
    p.softmax_lse = softmax_lse.data_ptr<float>();
    p.softmax_d = sd.data_ptr<float>();
    p.cu_seqlens_q = i32_ptr(cu_seqlens_q, q, "cu_seqlens_q");
    p.cu_seqlens_k = i32_ptr(cu_seqlens_k, q, "cu_seqlens_k");
    if (alibi_slopes.has_value()) {
        check_dev(*alibi_slopes, q, "alibi_slopes");
        TORCH_CHECK(alibi_slopes->scalar_type() == at::kFloat && alibi_slopes->stride(-1) == 1,
                    "ALiBi slopes must be fp32 with a contiguous last dimension");
        TORCH_CHECK(alibi_slopes->sizes() == at::IntArrayRef({H}) ||
                        alibi_slopes->sizes() == at::IntArrayRef({(int64_t)p.batch, H}),
                    "alibi_slopes must have shape (nheads) or (batch_size, nheads)");
        p.alibi_slopes = alibi_slopes->data_ptr<float>();
        p.alibi_batch_stride = alibi_slopes->dim() == 2 ? alibi_slopes->stride(0) : 0;
    }
    p.dropout_p = (float)p_dropout;
    p.softmax_scale = (float)softmax_scale;
    p.softcap = (float)softcap;
    p.is_causal = is_causal ? 1 : 0;
    p.window_size_left = (int32_t)window_size_left;
    p.window_size_right = (int32_t)window_size_right;
    p.deterministic = deterministic ? 1 : 0;
    p.attention_chunk = (int32_t)attention_chunk;
    check_status(fa_mha_varlen_bwd(&p, cur_stream()));
    return {dq, dk, dv, sd};
}

}  // namespace

TORCH_LIBRARY(fa_mi355x, m) {
    m.def(
        "fwd_kvcache(Tensor q, Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor? k, Tensor? v, Tensor? seqlens_k, "
        "Tensor? rotary_cos, Tensor? rotary_sin, Tensor? cache_batch_idx, Tensor? leftpad_k, Tensor? block_table, "
        "Tensor? alibi_slopes, float softmax_scale, bool is_causal, int window_size_left, int window_size_right, "
        "float softcap, bool is_rotary_interleaved, int num_splits) -> (Tensor, Tensor)");
    m.def(
        "fwd(Tensor q, Tensor k, Tensor v, Tensor? alibi_slopes, float p_dropout, float softmax_scale, bool is_causal, "
        "int window_size_left, int window_size_right, float softcap, int attention_chunk=0, Tensor? q_descale=None, "
        "Tensor? k_descale=None, Tensor? v_descale=None, int num_splits=0, Tensor(a!)? workspace=None, "
        "bool? pack_gqa=None) -> (Tensor, Tensor)");
    m.def(
        "fwd_kvcache_v3(Tensor q, Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor? k, Tensor? v, Tensor? seqlens_k, "
        "Tensor? rotary_cos, Tensor? rotary_sin, Tensor? cache_batch_idx, Tensor? leftpad_k, Tensor? block_table, "
        "Tensor? alibi_slopes, Tensor? cu_seqlens_q, Tensor? cu_seqlens_k_new, int max_seqlen_q, "
        "Tensor? rotary_seqlens, float softmax_scale, bool is_causal, int window_size_left, int window_size_right, "
        "int attention_chunk, float softcap, bool is_rotary_interleaved, int num_splits, Tensor? q_descale=None, "
        "Tensor? k_descale=None, Tensor? v_descale=None, Tensor(c!)? workspace=None, Tensor? qv=None, "
        "bool? pack_gqa=None) -> (Tensor, Tensor)");
    m.def(
        "varlen_fwd(Tensor q, Tensor k, Tensor v, Tensor cu_seqlens_q, Tensor? cu_seqlens_k, Tensor? seqused_k, "
        "Tensor? block_table, "
        "Tensor? alibi_slopes, int max_seqlen_q, int max_seqlen_k, float p_dropout, float softmax_scale, "
        "bool is_causal, int window_size_left, int window_size_right, float softcap, int attention_chunk=0, "
        "Tensor? q_descale=None, Tensor? k_descale=None, Tensor? v_descale=None, int num_splits=0, "
        "Tensor(a!)? workspace=None, bool? pack_gqa=None) -> (Tensor, Tensor)");
    m.def("fwd_combine(Tensor out_partial, Tensor lse_partial, ScalarType? out_dtype) -> (Tensor, Tensor)");
    m.def("fwd_combine_out(Tensor out_partial, Tensor lse_partial, Tensor(a!) out) -> Tensor");
    m.def(
        "bwd(Tensor dout, Tensor q, Tensor k, Tensor v, Tensor out, Tensor softmax_lse, Tensor? alibi_slopes, "
        "float p_dropout, float softmax_scale, bool is_causal, int window_size_left, int window_size_right, "
        "float softcap, bool deterministic, int attention_chunk=0) -> (Tensor, Tensor, Tensor, Tensor)");
    m.def(
        "varlen_bwd(Tensor dout, Tensor q, Tensor k, Tensor v, Tensor out, Tensor softmax_lse, Tensor cu_seqlens_q, "
        "Tensor cu_seqlens_k, Tensor? alibi_slopes, int max_seqlen_q, int max_seqlen_k, float p_dropout, "
        "float softmax_scale, bool is_causal, int window_size_left, int window_size_right, float softcap, "
        "bool deterministic, int attention_chunk=0) -> (Tensor, Tensor, Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(fa_mi355x, CUDA, m) {
    m.impl("fwd_kvcache", &fwd_kvcache);
    m.impl("fwd_kvcache_v3", &fwd_kvcache_v3);
    m.impl("fwd", &fwd);
    m.impl("varlen_fwd", &varlen_fwd);
    m.impl("fwd_combine", &fwd_combine);
    m.impl("fwd_combine_out", &fwd_combine_out);
    m.impl("bwd", &bwd);
    m.impl("varlen_bwd", &varlen_bwd);
}
