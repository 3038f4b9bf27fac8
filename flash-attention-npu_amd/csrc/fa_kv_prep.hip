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

// Element indices of pair p (0 <= p < D/2) and whether it is rotated.
__device__ __forceinline__ void pair_index(int p, int D, int rd, int interleaved, int& e1, int& e2, bool& rot,
                                           int& cs_idx) {
    if (rd > 0 && interleaved) {
        e1 = 2 * p;
        e2 = 2 * p + 1;
        rot = 2 * p < rd;
        cs_idx = p;
    } else if (rd > 0) {
        const int half = rd / 2;
        if (p < half) {
            e1 = p;
            e2 = p + half;
            rot = true;
            cs_idx = p;
        } else {
            e1 = rd + 2 * (p - half);
            e2 = e1 + 1;
            rot = false;
            cs_idx = 0;
        }
    } else {
        e1 = 2 * p;
        e2 = 2 * p + 1;
        rot = false;
        cs_idx = 0;
    }
}

// blockIdx.y: 0 = new keys, 1 = new values, 2 = q rotation.
template <int DT>
__global__ void __launch_bounds__(256) fa_kv_prep_kernel(KvPrepArgs a) {
    const int which = blockIdx.y;
    const int Dw = which == 1 ? a.Dv : a.D;
    const int pairs = Dw / 2;
    const int64_t nrows = which == 2 ? (int64_t)a.B * a.Sq * a.H : (int64_t)a.B * a.S_new * a.Hk;
    const int64_t total = nrows * pairs;
    const uint16_t* cs = static_cast<const uint16_t*>(a.cos);
    const uint16_t* sn = static_cast<const uint16_t*>(a.sin);
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int p = (int)(idx % pairs);
        const int64_t row = idx / pairs;
        int e1, e2, cs_idx;
        bool rot;
        const int rd = which == 1 ? 0 : a.rotary_dim;
        pair_index(p, Dw, rd, a.interleaved, e1, e2, rot, cs_idx);
        if (which == 2) {
            const int h = (int)(row % a.H);
            const int i = (int)((row / a.H) % a.Sq);
            const int b = (int)(row / ((int64_t)a.H * a.Sq));
            const uint16_t* src = static_cast<const uint16_t*>(a.q) + (int64_t)b * a.q_sb + (int64_t)i * a.q_si +
                                  (int64_t)h * a.q_sh;
            uint16_t* dst = static_cast<uint16_t*>(a.q_out) + (((int64_t)b * a.Sq + i) * a.H + h) * a.D;
            uint16_t x1 = src[e1], x2 = src[e2];
            if (rot) {
                int pos = (a.seqlens ? a.seqlens[b] : 0) + (a.q_same_pos ? 0 : i);
                pos = min(max(pos, 0), a.seqlen_ro - 1);
                float c = f16_to_32<DT>(cs[(int64_t)pos * a.cs_stride + cs_idx]);
                float s = f16_to_32<DT>(sn[(int64_t)pos * a.cs_stride + cs_idx]);
                float o1, o2;
                rope_pair<DT>(f16_to_32<DT>(x1), f16_to_32<DT>(x2), c, s, o1, o2);
                x1 = f32_to_16<DT>(o1);
                x2 = f32_to_16<DT>(o2);
            }
            dst[e1] = x1;
            dst[e2] = x2;
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
        uint16_t x1 = src[e1], x2 = src[e2];
        if (rot) {
            const int pos = min(j, a.seqlen_ro - 1);
            float c = f16_to_32<DT>(cs[(int64_t)pos * a.cs_stride + cs_idx]);
            float s = f16_to_32<DT>(sn[(int64_t)pos * a.cs_stride + cs_idx]);
            float o1, o2;
            rope_pair<DT>(f16_to_32<DT>(x1), f16_to_32<DT>(x2), c, s, o1, o2);
            x1 = f32_to_16<DT>(o1);
            x2 = f32_to_16<DT>(o2);
        }
        dst[e1] = x1;
        dst[e2] = x2;
    }
}

hipError_t launch_kv_prep(const KvPrepArgs& a, int dtype, hipStream_t stream) {
    const int parts = a.q_out ? 3 : 2;
    int64_t rows_kv = (int64_t)a.B * a.S_new * a.Hk;
    int64_t rows_q = a.q_out ? (int64_t)a.B * a.Sq * a.H : 0;
    int64_t mx = rows_kv > rows_q ? rows_kv : rows_q;
    int64_t work = mx * (a.D > a.Dv ? a.D : a.Dv) / 2;
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
