// fa_kv_prep.hip -- KV-cache front end for gfx950: in-place append of the new
// k/v tokens at cache_seqlens (contiguous or paged, through cache_batch_idx),
// rotary embedding on the new keys and on q.
//
// Semantics follow the flash_attn_with_kvcache docstring
// (flash_attn_npu_v2/interface_arch22.py:1452-1538 in the reference; the
// reference kernels accept k/v and cache_batch_idx but ignore them and reject
// rotary: csrc/arch22/flash_attn_npu_v2/flash_api.cpp:415-436):
//   cache[idx(b), L_b + t] = rope(k[b, t], pos = L_b + t),  t < S_new
//   q[b, i] rotated at L_b + i (causal or local) or at L_b (otherwise)
//   rotary_dim = 2 * cos.shape[1]; interleaved pairs (2i, 2i+1), GPT-NeoX pairs
//   (i, i + rotary_dim/2); dims >= rotary_dim are copied.
// Arithmetic: fp32 x1*c - x2*s and x2*c + x1*s with each product rounded to
// fp32 (contraction off), then round-to-nearest-even to the storage type, so
// the CPU checker reproduces every bit.
#include "fa_common.h"
#include "fa_kernel_args.h"

namespace fa {

#pragma clang fp contract(off)

template <int DT>
__device__ __forceinline__ void rope_pair(float x1, float x2, float c, float s, float& o1, float& o2) {
    float a = x1 * c;
    float bb = x2 * s;
    float cc = x2 * c;
    float dd = x1 * s;
    o1 = a - bb;
    o2 = cc + dd;
}

// Rotates 4 pairs (x1[e], x2[e]) with cos/sin entries cs_idx0 .. cs_idx0+3.
template <int DT>
__device__ __forceinline__ void rope4(uint16_t* x1, uint16_t* x2, const uint16_t* cs, const uint16_t* sn) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float o1, o2;
        rope_pair<DT>(f16_to_32<DT>(x1[e]), f16_to_32<DT>(x2[e]), f16_to_32<DT>(cs[e]), f16_to_32<DT>(sn[e]), o1, o2);
        x1[e] = f32_to_16<DT>(o1);
        x2[e] = f32_to_16<DT>(o2);
    }
}

// Moves (and, for keys and q, rotates) one 8-element unit u of a head row.
// GPT-NeoX: units u < rd/8 hold the 4 pairs (4u+e, 4u+e+rd/2); later units
// are the untouched dims rd + 8(u - rd/8) ... Interleaved: unit u holds the
// pairs (8u+2e, 8u+2e+1), rotated when 8u < rd. rd is a multiple of 16.
template <int DT>
__device__ __forceinline__ void move_unit(const uint16_t* src, uint16_t* dst, int u, int rd, int interleaved,
                                          const uint16_t* cs_row, const uint16_t* sn_row) {
    if (rd > 0 && !interleaved && u < rd / 8) {
        const int half = rd / 2;
        u32x2 a = *reinterpret_cast<const u32x2*>(src + 4 * u);
        u32x2 b = *reinterpret_cast<const u32x2*>(src + 4 * u + half);
        u32x2 c = *reinterpret_cast<const u32x2*>(cs_row + 4 * u);
        u32x2 s = *reinterpret_cast<const u32x2*>(sn_row + 4 * u);
        uint16_t x1[4], x2[4], cc[4], ss[4];
        __builtin_memcpy(x1, &a, 8);
        __builtin_memcpy(x2, &b, 8);
        __builtin_memcpy(cc, &c, 8);
        __builtin_memcpy(ss, &s, 8);
        rope4<DT>(x1, x2, cc, ss);
        __builtin_memcpy(&a, x1, 8);
        __builtin_memcpy(&b, x2, 8);
        *reinterpret_cast<u32x2*>(dst + 4 * u) = a;
        *reinterpret_cast<u32x2*>(dst + 4 * u + half) = b;
        return;
    }
    const int e0 = (rd > 0 && !interleaved) ? rd + 8 * (u - rd / 8) : 8 * u;
    u32x4 v = *reinterpret_cast<const u32x4*>(src + e0);
    if (rd > 0 && interleaved && e0 < rd) {
        uint16_t x[8], x1[4], x2[4];
        __builtin_memcpy(x, &v, 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x1[e] = x[2 * e];
            x2[e] = x[2 * e + 1];
        }
        u32x2 c = *reinterpret_cast<const u32x2*>(cs_row + 4 * u);
        u32x2 s = *reinterpret_cast<const u32x2*>(sn_row + 4 * u);
        uint16_t cc[4], ss[4];
        __builtin_memcpy(cc, &c, 8);
        __builtin_memcpy(ss, &s, 8);
        rope4<DT>(x1, x2, cc, ss);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[2 * e] = x1[e];
            x[2 * e + 1] = x2[e];
        }
        __builtin_memcpy(&v, x, 16);
    }
    *reinterpret_cast<u32x4*>(dst + e0) = v;
}

// blockIdx.y: 0 = new keys, 1 = new values, 2 = q rotation. One thread per
// 8-element unit (16-byte loads and stores).
template <int DT>
__global__ void __launch_bounds__(256) fa_kv_prep_kernel(KvPrepArgs a) {
    const int which = blockIdx.y;
    const int Dw = which == 1 ? a.Dv : a.D;
    const int units = Dw / 8;
    const int64_t nrows = which == 2 ? (int64_t)a.B * a.Sq * a.H : (int64_t)a.B * a.S_new * a.Hk;
    const int64_t total = nrows * units;
    const uint16_t* cs = static_cast<const uint16_t*>(a.cos);
    const uint16_t* sn = static_cast<const uint16_t*>(a.sin);
    const int rd = which == 1 ? 0 : a.rotary_dim;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int u = (int)(idx % units);
        const int64_t row = idx / units;
        if (which == 2) {
            const int h = (int)(row % a.H);
            const int i = (int)((row / a.H) % a.Sq);
            const int b = (int)(row / ((int64_t)a.H * a.Sq));
            const uint16_t* src = static_cast<const uint16_t*>(a.q) + (int64_t)b * a.q_sb + (int64_t)i * a.q_si +
                                  (int64_t)h * a.q_sh;
            uint16_t* dst = static_cast<uint16_t*>(a.q_out) + (((int64_t)b * a.Sq + i) * a.H + h) * a.D;
            int pos = (a.seqlens ? a.seqlens[b] : 0) + (a.q_same_pos ? 0 : i);
            pos = min(max(pos, 0), a.seqlen_ro - 1);
            move_unit<DT>(src, dst, u, rd, a.interleaved, cs + (int64_t)pos * a.cs_stride, sn + (int64_t)pos * a.cs_stride);
            continue;
        }
        const int h = (int)(row % a.Hk);
        const int t = (int)((row / a.Hk) % a.S_new);
        const int b = (int)(row / ((int64_t)a.Hk * a.S_new));
        const int j = a.seqlens[b] + t;
        if (j < 0 || j >= a.kv_capacity) continue;  // cache too small: nothing is written
        const int crow = a.batch_idx ? a.batch_idx[b] : b;
        uint16_t* cache = static_cast<uint16_t*>(which == 0 ? a.k_cache : a.v_cache);
        const int64_t sb = which == 0 ? a.k_sb : a.v_sb, si = which == 0 ? a.k_si : a.v_si,
                      sh = which == 0 ? a.k_sh : a.v_sh;
        uint16_t* dst;
        if (a.block_table) {
            if (crow < 0 || crow >= a.bt_rows) continue;
            int blk = a.block_table[(int64_t)crow * a.bt_stride + j / a.page];
            if (blk < 0 || blk >= a.num_blocks) continue;
            dst = cache + (int64_t)blk * sb + (int64_t)(j % a.page) * si + (int64_t)h * sh;
        } else {
            if (crow < 0 || crow >= a.batch_cache) continue;
            dst = cache + (int64_t)crow * sb + (int64_t)j * si + (int64_t)h * sh;
        }
        const uint16_t* src;
        if (which == 0)
            src = static_cast<const uint16_t*>(a.k_new) + (int64_t)b * a.kn_sb + (int64_t)t * a.kn_si +
                  (int64_t)h * a.kn_sh;
        else
            src = static_cast<const uint16_t*>(a.v_new) + (int64_t)b * a.vn_sb + (int64_t)t * a.vn_si +
                  (int64_t)h * a.vn_sh;
        const int pos = min(j, a.seqlen_ro - 1);
        move_unit<DT>(src, dst, u, rd, a.interleaved, rd ? cs + (int64_t)pos * a.cs_stride : nullptr,
                      rd ? sn + (int64_t)pos * a.cs_stride : nullptr);
    }
}

hipError_t launch_kv_prep(const KvPrepArgs& a, int dtype, hipStream_t stream) {
    const int parts = a.q_out ? 3 : 2;
    int64_t rows_kv = (int64_t)a.B * a.S_new * a.Hk;
    int64_t rows_q = a.q_out ? (int64_t)a.B * a.Sq * a.H : 0;
    int64_t mx = rows_kv > rows_q ? rows_kv : rows_q;
    int64_t work = mx * (a.D > a.Dv ? a.D : a.Dv) / 8;
    int grid = (int)((work + 255) / 256);
    if (grid > 8192) grid = 8192;
    if (grid < 1) grid = 1;
    // rotary is only defined together with an append, so no new tokens means no work
    if (!(a.k_new && a.S_new > 0)) return hipSuccess;
    const int ny = parts;
    if (dtype == DT_BF16)
        hipLaunchKernelGGL(fa_kv_prep_kernel<DT_BF16>, dim3(grid, ny), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(fa_kv_prep_kernel<DT_FP16>, dim3(grid, ny), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace fa
