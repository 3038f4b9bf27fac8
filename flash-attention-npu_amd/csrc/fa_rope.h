// fa_rope.h -- rotary embedding of one 8-element chunk of a head row, shared
// by the append kernel (new keys, decode q) and the prefill kernel's q load.
//
// Semantics (flash_attn_with_kvcache docstring, flash_attn_npu_v2/
// interface_arch22.py:1452-1538 in the reference): rotary_dim rd = 2 *
// cos.shape[1], a multiple of 16; dims >= rd are untouched.
//   GPT-NeoX: pair (i, i + rd/2), i < rd/2, angle index i.
//   interleaved: pair (2i, 2i + 1), angle index i.
//   x1' = x1*c - x2*s,  x2' = x2*c + x1*s
// Each product is rounded to fp32 (contraction off) before the add, then the
// sum is rounded to nearest-even in the storage type, so a CPU restatement
// reproduces every bit.
#pragma once
#include "fa_common.h"

namespace fa {

__device__ __forceinline__ u32x4 load_u32x4_a8(const uint16_t* p) {
    const u32x2 lo = *reinterpret_cast<const u32x2*>(p);
    const u32x2 hi = *reinterpret_cast<const u32x2*>(p + 4);
    return u32x4{lo.x, lo.y, hi.x, hi.y};
}

// The operands of chunk c (dims 8c .. 8c+7, 8c < rd) besides the chunk
// itself: in NeoX form a chunk lies wholly in one half (rd/2 is a multiple of
// 8) and pairs with the chunk rd/2 away; interleaved pairs lie inside the
// chunk and need 4 angles. cs_row / sn_row point at the position's cos / sin
// row (rd/2 entries, 8-byte aligned). Loading and rotating are separate so a
// caller can issue these loads early and rotate later.
struct RopeOps {
    u32x4 partner, cs, sn;
};

__device__ __forceinline__ RopeOps rope_load(const uint16_t* row, int c, int rd, bool interleaved,
                                             const uint16_t* cs_row, const uint16_t* sn_row) {
    RopeOps o;
    if (interleaved) {
        const u32x2 cw = *reinterpret_cast<const u32x2*>(cs_row + 4 * c);
        const u32x2 sw = *reinterpret_cast<const u32x2*>(sn_row + 4 * c);
        o.partner = u32x4{0u, 0u, 0u, 0u};
        o.cs = u32x4{cw.x, cw.y, 0u, 0u};
        o.sn = u32x4{sw.x, sw.y, 0u, 0u};
    } else {
        const int half = rd >> 1;
        const bool first = 8 * c < half;
        const int pc = first ? 8 * c + half : 8 * c - half;  // partner chunk's first dim
        const int ci = first ? 8 * c : 8 * c - half;          // angle index of element 0
        o.partner = *reinterpret_cast<const u32x4*>(row + pc);
        o.cs = load_u32x4_a8(cs_row + ci);
        o.sn = load_u32x4_a8(sn_row + ci);
    }
    return o;
}

// Chunk c of the row after rotation; x is that chunk as loaded.
template <int DT>
__device__ __forceinline__ u32x4 rope_apply(u32x4 x, const RopeOps& op, int c, int rd, bool interleaved) {
#pragma clang fp contract(off)
    uint16_t xv[8], ov[8], cc[8], ss[8];
    __builtin_memcpy(xv, &x, 16);
    __builtin_memcpy(cc, &op.cs, 16);
    __builtin_memcpy(ss, &op.sn, 16);
    if (interleaved) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float x1 = f16_to_32<DT>(xv[2 * e]), x2 = f16_to_32<DT>(xv[2 * e + 1]);
            const float co = f16_to_32<DT>(cc[e]), si = f16_to_32<DT>(ss[e]);
            const float a = x1 * co, b = x2 * si, d = x2 * co, f = x1 * si;
            ov[2 * e] = f32_to_16<DT>(a - b);
            ov[2 * e + 1] = f32_to_16<DT>(d + f);
        }
    } else {
        const bool first = 8 * c < (rd >> 1);
        uint16_t pv[8];
        __builtin_memcpy(pv, &op.partner, 16);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float xo = f16_to_32<DT>(xv[e]), xp = f16_to_32<DT>(pv[e]);
            const float co = f16_to_32<DT>(cc[e]), si = f16_to_32<DT>(ss[e]);
            const float a = xo * co, b = xp * si;
            ov[e] = f32_to_16<DT>(first ? a - b : a + b);
        }
    }
    u32x4 o;
    __builtin_memcpy(&o, ov, 16);
    return o;
}

template <int DT>
__device__ __forceinline__ u32x4 rope_chunk(u32x4 x, const uint16_t* row, int c, int rd, bool interleaved,
                                            const uint16_t* cs_row, const uint16_t* sn_row) {
    return rope_apply<DT>(x, rope_load(row, c, rd, interleaved, cs_row, sn_row), c, rd, interleaved);
}

}  // namespace fa
