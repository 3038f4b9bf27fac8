// fa_kv_prep.hip -- KV-cache front end for gfx950: in-place append of the new
// k/v tokens at cache_seqlens (contiguous or paged, through cache_batch_idx),
// rotary embedding on the new keys and, for decode, on q.
//
// Semantics follow the flash_attn_with_kvcache docstring
// (flash_attn_npu_v2/interface_arch22.py:1452-1538 in the reference; the
// reference kernels accept k/v and cache_batch_idx but ignore them and reject
// rotary: csrc/arch22/flash_attn_npu_v2/flash_api.cpp:415-436):
//   cache[idx(b), L_b + t] = rope(k[b, t], pos = P_b + t),  t < S_new(b)
//   q[b, i] rotated at P_b + i (causal or local) or at P_b (otherwise)
// with P_b = rotary_seqlens[b] when given, else L_b (the v3 docstring,
// README.md:311-401 of the reference). New tokens and q may be ragged
// ((total, heads, D) split by cu_seqlens_k_new / cu_seqlens_q).
// The rotation itself is rope_chunk (fa_rope.h). Prefill rotates q inside
// its own q load, so only decode asks for q_out here.
#include "fa_common.h"
#include "fa_kernel_args.h"
#include "fa_rope.h"

#include <type_traits>

namespace fa {

// blockIdx.y: 0 = new keys, 1 = new values, 2 = q rotation. A workgroup
// covers 256 / U head rows (U = 16-byte chunks per row), one thread per chunk:
// every thread moves 16 bytes, and all index arithmetic is 32-bit (the host
// keeps row counts below 2^31). DT_FP8 rows are e4m3fn bytes, copied as they
// are (the host admits no rotary with FP8).
template <int DT>
__global__ void __launch_bounds__(256) fa_kv_prep_kernel(KvPrepArgs a) {
    constexpr bool F8 = DT == DT_FP8;
    using ET = std::conditional_t<F8, uint8_t, uint16_t>;
    constexpr int EPL = 16 / sizeof(ET);  // elements per 16-byte chunk
    const int which = blockIdx.y;
    const int U = (which == 1 ? a.Dv : a.D) / EPL;
    const int rpb = 256 / U;
    const int tid = threadIdx.x;
    const int rl = tid / U;
    const int u = tid - rl * U;
    if (rl >= rpb) return;
    const int row = blockIdx.x * rpb + rl;
    const int rd = (which == 1 || F8) ? 0 : a.rotary_dim;
    const uint16_t* cs = static_cast<const uint16_t*>(a.cos);
    const uint16_t* sn = static_cast<const uint16_t*>(a.sin);

    const ET* src;
    ET* dst;
    int pos;
    if (which == 2) {
        const int h = row % a.H;
        const int bi = row / a.H;
        int b, i;
        if (a.cu_q) {  // ragged q: row bi of (total_q, H, D)
            if (row >= a.total_q * a.H) return;
            b = seq_of(a.cu_q, a.B, bi);
            i = bi - a.cu_q[b];
            src = static_cast<const ET*>(a.q) + (int64_t)bi * a.q_si + (int64_t)h * a.q_sh;
        } else {
            if (row >= a.B * a.Sq * a.H) return;
            i = bi % a.Sq;
            b = bi / a.Sq;
            src = static_cast<const ET*>(a.q) + (int64_t)b * a.q_sb + (int64_t)i * a.q_si + (int64_t)h * a.q_sh;
        }
        dst = static_cast<ET*>(a.q_out) + (int64_t)row * a.D;
        pos = (a.rot_pos ? a.rot_pos[b] : a.seqlens ? a.seqlens[b] : 0) + (a.q_same_pos ? 0 : i);
    } else {
        const int h = row % a.Hk;
        const int bt = row / a.Hk;
        int b, t;
        int64_t src_off;
        if (a.cu_knew) {  // ragged new tokens: row bt of (total_new, Hk, D)
            if (row >= a.total_new * a.Hk) return;
            b = seq_of(a.cu_knew, a.B, bt);
            t = bt - a.cu_knew[b];
            src_off = (int64_t)bt * (which == 0 ? a.kn_si : a.vn_si);
        } else {
            if (row >= a.B * a.S_new * a.Hk) return;
            t = bt % a.S_new;
            b = bt / a.S_new;
            src_off = which == 0 ? (int64_t)b * a.kn_sb + (int64_t)t * a.kn_si : (int64_t)b * a.vn_sb + (int64_t)t * a.vn_si;
        }
        const int j = a.seqlens[b] + t;
        if (j < 0 || j >= a.kv_capacity) return;  // cache too small: nothing is written
        const int crow = a.batch_idx ? a.batch_idx[b] : b;
        ET* cache = static_cast<ET*>(which == 0 ? a.k_cache : a.v_cache);
        const int64_t sb = which == 0 ? a.k_sb : a.v_sb, si = which == 0 ? a.k_si : a.v_si,
                      sh = which == 0 ? a.k_sh : a.v_sh;
        if (a.block_table) {
            if (crow < 0 || crow >= a.bt_rows) return;
            const int blk = a.block_table[(int64_t)crow * a.bt_stride + j / a.page];
            if (blk < 0 || blk >= a.num_blocks) return;
            dst = cache + (int64_t)blk * sb + (int64_t)(j % a.page) * si + (int64_t)h * sh;
        } else {
            if (crow < 0 || crow >= a.batch_cache) return;
            dst = cache + (int64_t)crow * sb + (int64_t)j * si + (int64_t)h * sh;
        }
        src = which == 0 ? static_cast<const ET*>(a.k_new) + src_off + (int64_t)h * a.kn_sh
                         : static_cast<const ET*>(a.v_new) + src_off + (int64_t)h * a.vn_sh;
        pos = a.rot_pos ? a.rot_pos[b] + t : j;
    }
    u32x4 x = *reinterpret_cast<const u32x4*>(src + EPL * u);
    if constexpr (!F8) {
        if (8 * u < rd) {
            pos = min(max(pos, 0), a.seqlen_ro - 1);
            x = rope_chunk<DT>(x, src, u, rd, a.interleaved != 0, cs + (int64_t)pos * a.cs_stride,
                               sn + (int64_t)pos * a.cs_stride);
        }
    }
    *reinterpret_cast<u32x4*>(dst + EPL * u) = x;
}

hipError_t launch_kv_prep(const KvPrepArgs& a, int dtype, hipStream_t stream) {
    const int64_t rows_kv = !a.k_new ? 0 : a.cu_knew ? (int64_t)a.total_new * a.Hk : (int64_t)a.B * a.S_new * a.Hk;
    const int64_t rows_q = !a.q_out ? 0 : a.cu_q ? (int64_t)a.total_q * a.H : (int64_t)a.B * a.Sq * a.H;
    if (rows_kv >= INT32_MAX || rows_q >= INT32_MAX) return hipErrorInvalidValue;
    const int rpb = 256 / ((a.D > a.Dv ? a.D : a.Dv) / (dtype == DT_FP8 ? 16 : 8));
    const int64_t mx = rows_kv > rows_q ? rows_kv : rows_q;
    if (mx == 0) return hipSuccess;
    const int grid = (int)((mx + rpb - 1) / rpb);
    const int ny = a.q_out ? 3 : 2;
    if (dtype == DT_BF16)
        hipLaunchKernelGGL(fa_kv_prep_kernel<DT_BF16>, dim3(grid, ny), dim3(256), 0, stream, a);
    else if (dtype == DT_FP8)
        hipLaunchKernelGGL(fa_kv_prep_kernel<DT_FP8>, dim3(grid, ny), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(fa_kv_prep_kernel<DT_FP16>, dim3(grid, ny), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace fa
