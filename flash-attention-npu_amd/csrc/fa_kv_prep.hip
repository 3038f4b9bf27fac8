// fa_kv_prep.hip -- KV-cache front end for gfx950: in-place append of the new
// k/v tokens at cache_seqlens (contiguous or paged, through cache_batch_idx),
// rotary embedding on the new keys and, for decode, on q.
//
// Semantics follow the flash_attn_with_kvcache docstring
// (flash_attn_npu_v2/interface_arch22.py:1452-1538 in the reference; the
// reference kernels accept k/v and cache_batch_idx but ignore them and reject
// rotary: csrc/arch22/flash_attn_npu_v2/flash_api.cpp:415-436):
//   cache[idx(b), L_b + t] = rope(k[b, t], pos = L_b + t),  t < S_new
//   q[b, i] rotated at L_b + i (causal or local) or at L_b (otherwise)
// The rotation itself is rope_chunk (fa_rope.h). Prefill rotates q inside
// its own q load, so only decode asks for q_out here.
#include "fa_common.h"
#include "fa_kernel_args.h"
#include "fa_rope.h"

namespace fa {

// blockIdx.y: 0 = new keys, 1 = new values, 2 = q rotation. A workgroup
// covers 256 / U head rows (U = 16-byte chunks per row), one thread per chunk:
// every thread moves 16 bytes, and all index arithmetic is 32-bit (the host
// keeps row counts below 2^31).
template <int DT>
__global__ void __launch_bounds__(256) fa_kv_prep_kernel(KvPrepArgs a) {
    const int which = blockIdx.y;
    const int U = (which == 1 ? a.Dv : a.D) >> 3;
    const int rpb = 256 / U;
    const int tid = threadIdx.x;
    const int rl = tid / U;
    const int u = tid - rl * U;
    if (rl >= rpb) return;
    const int row = blockIdx.x * rpb + rl;
    const int rd = which == 1 ? 0 : a.rotary_dim;
    const uint16_t* cs = static_cast<const uint16_t*>(a.cos);
    const uint16_t* sn = static_cast<const uint16_t*>(a.sin);

    const uint16_t* src;
    uint16_t* dst;
    int pos;
    if (which == 2) {
        if (row >= a.B * a.Sq * a.H) return;
        const int h = row % a.H;
        const int bi = row / a.H;
        const int i = bi % a.Sq;
        const int b = bi / a.Sq;
        src = static_cast<const uint16_t*>(a.q) + (int64_t)b * a.q_sb + (int64_t)i * a.q_si + (int64_t)h * a.q_sh;
        dst = static_cast<uint16_t*>(a.q_out) + (int64_t)row * a.D;
        pos = (a.seqlens ? a.seqlens[b] : 0) + (a.q_same_pos ? 0 : i);
    } else {
        if (row >= a.B * a.S_new * a.Hk) return;
        const int h = row % a.Hk;
        const int bt = row / a.Hk;
        const int t = bt % a.S_new;
        const int b = bt / a.S_new;
        const int j = a.seqlens[b] + t;
        if (j < 0 || j >= a.kv_capacity) return;  // cache too small: nothing is written
        const int crow = a.batch_idx ? a.batch_idx[b] : b;
        uint16_t* cache = static_cast<uint16_t*>(which == 0 ? a.k_cache : a.v_cache);
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
        src = which == 0 ? static_cast<const uint16_t*>(a.k_new) + (int64_t)b * a.kn_sb + (int64_t)t * a.kn_si +
                               (int64_t)h * a.kn_sh
                         : static_cast<const uint16_t*>(a.v_new) + (int64_t)b * a.vn_sb + (int64_t)t * a.vn_si +
                               (int64_t)h * a.vn_sh;
        pos = j;
    }
    u32x4 x = *reinterpret_cast<const u32x4*>(src + 8 * u);
    if (8 * u < rd) {
        pos = min(max(pos, 0), a.seqlen_ro - 1);
        x = rope_chunk<DT>(x, src, u, rd, a.interleaved != 0, cs + (int64_t)pos * a.cs_stride,
                           sn + (int64_t)pos * a.cs_stride);
    }
    *reinterpret_cast<u32x4*>(dst + 8 * u) = x;
}

hipError_t launch_kv_prep(const KvPrepArgs& a, int dtype, hipStream_t stream) {
    const int64_t rows_kv = a.k_new ? (int64_t)a.B * a.S_new * a.Hk : 0;
    const int64_t rows_q = a.q_out ? (int64_t)a.B * a.Sq * a.H : 0;
    if (rows_kv >= INT32_MAX || rows_q >= INT32_MAX) return hipErrorInvalidValue;
    const int rpb = 256 / ((a.D > a.Dv ? a.D : a.Dv) >> 3);
    const int64_t mx = rows_kv > rows_q ? rows_kv : rows_q;
    if (mx == 0) return hipSuccess;
    const int grid = (int)((mx + rpb - 1) / rpb);
    const int ny = a.q_out ? 3 : 2;
    if (dtype == DT_BF16)
        hipLaunchKernelGGL(fa_kv_prep_kernel<DT_BF16>, dim3(grid, ny), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(fa_kv_prep_kernel<DT_FP16>, dim3(grid, ny), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace fa
