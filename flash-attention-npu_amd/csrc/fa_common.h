// fa_common.h -- device-side types and helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

// DT_FP8: OCP e4m3fn inputs, widened to bf16 on load; bf16 arithmetic and
// output (the value matches FA_DTYPE_FP8_E4M3).
enum : int { DT_FP16 = 0, DT_BF16 = 1, DT_FP8 = 3 };

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// 16x16x32 MFMA on 16-byte packed operands. Lane l holds A[l%16][8*(l/16)+e]
// and B[8*(l/16)+e][l%16]; the result lane l holds D[4*(l/16)+i][l%16].
// DT_FP8 operands are already widened to bf16.
template <int DT>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (DT == DT_FP16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
}

// Round-to-nearest-even conversions of 8 floats into one 16-byte operand
// (bf16 for DT_BF16 and DT_FP8).
template <int DT>
__device__ __forceinline__ u32x4 pack8(f32x8 v) {
    if constexpr (DT == DT_FP16) {
        f16x8 h = __builtin_convertvector(v, f16x8);
        return __builtin_bit_cast(u32x4, h);
    } else {
        bf16x8 h = __builtin_convertvector(v, bf16x8);
        return __builtin_bit_cast(u32x4, h);
    }
}

template <int DT>
__device__ __forceinline__ uint16_t f32_to_16(float f) {
    if constexpr (DT == DT_FP16) {
        return __builtin_bit_cast(uint16_t, (_Float16)f);
    } else {
        return __builtin_bit_cast(uint16_t, (__bf16)f);
    }
}

template <int DT>
__device__ __forceinline__ float f16_to_32(uint16_t h) {
    if constexpr (DT == DT_FP16) {
        return (float)__builtin_bit_cast(_Float16, h);
    } else {
        return __builtin_bit_cast(float, (uint32_t)h << 16);
    }
}

// 8 e4m3fn values (the bytes of r, lowest first) -> 8 bf16 in one 16-byte
// operand. Exact: every e4m3fn value (normal, subnormal, +-0, NaN) is a bf16
// value, and the scale is 1.
__device__ __forceinline__ u32x4 fp8x8_to_bf16(u32x2 r) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    u32x4 o;
    o[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)r[0], 1.0f, false));
    o[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)r[0], 1.0f, true));
    o[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)r[1], 1.0f, false));
    o[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)r[1], 1.0f, true));
    return o;
}

// 16x16x128 MFMA on e4m3 operands (gfx950 f8f6f4, format 0 = E4M3 for both,
// E8M0 scales 127 = 1). Lane l holds A[l%16][32*(l/16)+e] and
// B[32*(l/16)+e][l%16], e < 32: the 32 bytes of a[0], a[1] (lowest first).
// The result lane l holds D[4*(l/16)+i][l%16]. Products of e4m3 values are
// exact in fp32.
__device__ __forceinline__ f32x4 mfma16x16x128_e4m3(u32x4 a0, u32x4 a1, u32x4 b0, u32x4 b1, f32x4 c) {
    typedef int i32x8 __attribute__((ext_vector_type(8)));
    const i32x8 a = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
    const i32x8 b = {(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// FP8 descale factor of (batch b, kv head hk); a null table means 1.
__device__ __forceinline__ float descale_at(const float* p, int64_t sb, int64_t sh, int b, int hk) {
    return p ? p[(int64_t)b * sb + (int64_t)hk * sh] : 1.f;
}

// LDS tile swizzles (16-byte chunk c of row r): swz_k keeps 16 consecutive
// rows' row reads (one chunk each) on distinct banks; swz_v does the same for
// the ds_read_b64_tr_b16 transpose reads of 4-row groups.
__device__ __forceinline__ int swz_k(int r, int c) { return c ^ (r & 15); }
__device__ __forceinline__ int swz_v(int r, int c) { return c ^ ((r & 3) << 1) ^ (((r >> 2) & 1) << 3); }
// The same for 128-byte rows (head dim 64, 8 chunks): row r starts at bank
// 32 * (r & 1), so the XOR comes from the row bits above the parity. K: the 16
// rows of a 16-byte operand read hit 16 different 4-bank groups. V: the 8 rows
// a half wave of transpose reads covers take 4 disjoint chunk pairs per parity.
__device__ __forceinline__ int swz_k64(int r, int c) { return c ^ ((r >> 1) & 7); }
__device__ __forceinline__ int swz_v64(int r, int c) { return c ^ (((r >> 1) & 3) << 1); }
// 128-byte rows read both ways (row reads of 16 rows and transpose reads of 8
// rows by a half wave): the XOR f(x) = ((x & 3) << 1) | (x >> 2) of x = r >> 1
// is a bijection on 0..7 (16 distinct 4-bank groups for a row read) and gives
// rows 0..7 chunk pairs 0, 2, 4, 6 apart (disjoint for a transpose read).
__device__ __forceinline__ int swz_b64(int r, int c) {
    const int x = (r >> 1) & 7;
    return c ^ (((x & 3) << 1) | (x >> 2));
}

// 256-byte rows (head dim 128) kept as 8-byte halves, for tiles read both by
// rows as 16x16x32 operands (two ds_read_b64 per operand: ds_read_b128 peaks
// at half the LDS rate of ds_read_b64 on this part) and transposed with
// ds_read_b64_tr_b16. Half h of 16-byte chunk c of row r sits in plane
// h ^ ((c >> 2) & 1) (the two 128-byte halves of the row), slot
// (c ^ pi(r)) & 15 with pi(r) = ((r & 7) << 1) | ((r >> 3) & 1). A row read
// (lane li of group G: row li, chunk 4G + s, one half) puts groups 0 / 1 (2 /
// 3) in different planes and 16 rows on 16 slots; a transpose read (rows
// 4G + (li >> 2), chunks 2d, 2d + 1, half li & 1) puts the halves in different
// planes and 8 rows x 2 chunks on 16 slots, since pi(0..7) and pi(8..15)
// differ in their upper three bits. Either way 32 lanes cover the 64 banks.
// Returns the element offset.
// LDS byte address of a __shared__ element, and an 8-byte LDS load from one
__device__ __forceinline__ unsigned lds_addr(const void* p) {
    return (unsigned)(size_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ u32x2 lds_load_u32x2(unsigned a) {
    return *(const __attribute__((address_space(3))) u32x2*)(size_t)a;
}
__device__ __forceinline__ int split_addr128(int r, int c, int h) {
    const int pi = ((r & 7) << 1) | ((r >> 3) & 1);
    return r * 128 + ((h ^ (c >> 2)) & 1) * 64 + ((c ^ pi) & 15) * 4;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }
// tanh(z) = 1 - 2 / (e^(2z) + 1) on the hardware exp2 and reciprocal: absolute
// error ~1e-7 over the whole range, +-1 exactly once e^(2z) over- or underflows
// (|z| > ~44); used for the soft cap, where cap * tanh enters exp() as an
// absolute score, so an absolute error of cap * 1e-7 is what matters.
__device__ __forceinline__ float fast_tanh(float z) {
    const float e = fast_exp2(z * (2.f * kLog2e));
    return 1.f - 2.f * __builtin_amdgcn_rcpf(e + 1.f);
}

__device__ __forceinline__ float wave_max16x4(float v) {
    // max over the 4 lanes l, l^16, l^32, l^48 that hold the same MFMA column
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}

__device__ __forceinline__ float wave_sum16x4(float v) {
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

// Sequence of ragged row T: the largest b < B with cu[b] <= T (cu is a
// non-decreasing prefix of B + 1 entries).
__device__ __forceinline__ int seq_of(const int* cu, int B, int T) {
    int lo = 0, hi = B;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (cu[mid] <= T) lo = mid;
        else hi = mid;
    }
    return lo;
}

// First key of the attention chunk that holds diagonal position p (chunk > 0):
// chunk * floor(p / chunk), also for negative p.
__device__ __forceinline__ int chunk_start(int p, int chunk) {
    const int q = p >= 0 ? p / chunk : -((-p + chunk - 1) / chunk);
    return q * chunk;
}

// Keys visible to the query whose diagonal position is d (d = i + Sk - Sq,
// bottom-right aligned) are [key_lo(d), key_hi(d)] intersected with [0, Sk):
// the local window (wl / wr, -1 = unbounded, causal is wr = 0) and, with
// attention_chunk c > 0, the chunk [chunk_start(d), chunk_start(d) + c).
// Both bounds are non-decreasing in d, so a run of rows sees at most
// [key_lo(first row), key_hi(last row)].
__device__ __forceinline__ int key_lo(int d, int wl, int chunk) {
    int lo = wl >= 0 ? d - wl : -0x3fffffff;
    if (chunk > 0) lo = max(lo, chunk_start(d, chunk));
    return lo;
}
__device__ __forceinline__ int key_hi(int d, int wr, int chunk) {
    int hi = wr >= 0 ? d + wr : 0x3fffffff;
    if (chunk > 0) hi = min(hi, chunk_start(d, chunk) + chunk - 1);
    return hi;
}

// The inverse view: key j is visible to the queries whose diagonal position d
// lies in [row_lo(j), row_hi(j)] (non-decreasing in j as well).
__device__ __forceinline__ int row_lo(int j, int wr, int chunk) {
    int lo = wr >= 0 ? j - wr : -0x3fffffff;
    if (chunk > 0) lo = max(lo, chunk_start(j, chunk));
    return lo;
}
__device__ __forceinline__ int row_hi(int j, int wl, int chunk) {
    int hi = wl >= 0 ? j + wl : 0x3fffffff;
    if (chunk > 0) hi = min(hi, chunk_start(j, chunk) + chunk - 1);
    return hi;
}

}  // namespace fa
