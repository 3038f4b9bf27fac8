// fa_bwd.hip -- FlashAttention backward (dense / varlen) for gfx950 (MI355X).
//
// Reference behaviour being reproduced (paths relative to the reference repo):
//   mha_bwd / mha_varlen_bwd       csrc/arch22/flash_attn_npu_v2/flash_api.cpp:1063-1299
//   FAG kernel (launch_fag_general) csrc/arch22/flash_attn_npu_v2/fag_general_host.cpp
//   golden                          tests/fa_small_op_golden.py:85-353
// Given q, k, v, out, dout and the forward's log-sum-exp, with P recomputed as
// exp(s - lse) (s the scaled, optionally soft-capped and ALiBi-biased score):
//   dsum_i = sum_d dout[i,d] * out[i,d]
//   dV = P^T dout,  dP = dout V^T,  dS = P * (dP - dsum) * scale [* (1 - tanh^2)]
//   dQ = dS K,      dK = dS^T Q
// (the golden's rowsum(dP * P) equals dsum up to the rounding of out).
//
// MI355X design: two launches, no atomics, so results are deterministic.
//   * fa_bwd_dq_kernel runs first and also computes dsum for its rows (from
//     the out rows and the dout rows it loads anyway), writing it for the
//     dK/dV kernel and as the returned softmax_d.
//   * fa_bwd_dkdv_kernel: one workgroup per (batch, kv head, 128-key block);
//     each of 8 waves keeps 16 keys' K and V in registers as MFMA B operands
//     and streams the packed (query, head) rows of all g query heads through
//     double-buffered LDS tiles of 64 rows. S = Q.K^T and dP = dO.V^T land
//     with one key and 8 rows per lane, exactly the packed operand of
//     dV^T += dO^T.P and dK^T += Q^T.dS, whose dO^T / Q^T operands are
//     transpose reads (ds_read_b64_tr_b16) of the same tiles. GQA needs no
//     reduction: the g heads of a kv head are rows of the same work item.
//   * fa_bwd_dq_kernel: the forward's shape (8 waves x 16 packed rows, 64-key
//     LDS tiles): S^T = K.Q^T and dP^T = V.dO^T with q and dout in registers,
//     then dQ^T += K^T.dS^T with K^T by transpose reads.
// dS and P are rounded to the input type before their MFMAs.
#include "fa_common.h"
#include "fa_kernel_args.h"
#include "fa_udiv.h"

#include <type_traits>

namespace fa {

namespace bw {
constexpr int kMaxBatch = 2048;
}  // namespace bw

// Tile shapes per kernel head dim (128 or 256).
template <int HD>
struct BwCfg {
    static constexpr int D = HD;
    static constexpr int DCH = D / 8;
    static constexpr int KSTEPS = D / 32;
    static constexpr int DBLK = D / 16;
    // dK/dV kernel: 16 keys per wave, q tiles of 64 packed rows. At 256 the
    // K/V operands and dK^T/dV^T accumulators of a wave take ~200 registers,
    // so the kernel runs one wave per SIMD (4 waves, MFMA accumulators in the
    // accumulation registers).
    static constexpr int KNW = HD > 128 ? 4 : 8;
    static constexpr int KRB = HD > 128 ? 1 : HD == 64 ? 2 : 1;  // 16-key blocks per wave
    static constexpr int KNT = KNW * 64;
    static constexpr int BK = KNW * 16 * KRB;
    static constexpr int BQ = 64;
    static constexpr int CPQ = BQ * DCH / KNT;  // chunks per thread per q (and dout) tile
    // dQ kernel: 2 row blocks of 16 per wave up to head dim 128, so every
    // K / V operand read from LDS feeds twice the products (the kernel is
    // bound by LDS reads: 3053 -> 2762 us for the whole backward of B4 S4096
    // H32/8 causal; the BIAS instance spills a few values at 128); 8 waves
    // and 64-key tiles up to 128, one wave per SIMD, 1 row block and 32-key
    // tiles at 256
    static constexpr int QNW = HD > 128 ? 4 : 8;
    static constexpr int QNT = QNW * 64;
    static constexpr int RB = HD <= 128 ? 2 : 1;
    static constexpr int BM = QNW * RB * 16;
    static constexpr int BN = HD > 128 ? 32 : 64;
    static constexpr int CPK = BN * DCH / QNT;
};

struct BwBatch {
    int sq, sk, rows;  // query positions, keys, packed rows (sq * g)
};

__device__ __forceinline__ BwBatch bw_batch(const BwdArgs& a, int b) {
    BwBatch r;
    int sq = a.cu_seqlens_q ? a.cu_seqlens_q[b + 1] - a.cu_seqlens_q[b] : a.Sq;
    int sk = a.cu_seqlens_k ? a.cu_seqlens_k[b + 1] - a.cu_seqlens_k[b] : a.Sk;
    r.sq = min(max(sq, 0), a.Sq);
    r.sk = min(max(sk, 0), a.Sk);
    r.rows = r.sq * a.g;
    return r;
}

// Per-batch item prefix in LDS (s_pref[0..B]); items(b) is the work item
// count of batch b. Every workgroup computes the same table.
template <int NT, class F>
__device__ __forceinline__ int bw_prefix(const BwdArgs& a, int* s_pref, F items) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int b = tid; b < a.B; b += NT) s_pref[b + 1] = items(b);
    __syncthreads();
    if (wave == 0) {
        const int seg = (a.B + 63) / 64, b0 = lane * seg;
        int local = 0;
        for (int k = 0; k < seg; ++k)
            if (b0 + k < a.B) local += s_pref[b0 + k + 1];
        int incl = local;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            int v = __shfl_up(incl, o);
            if (lane >= o) incl += v;
        }
        int run = incl - local;
        for (int k = 0; k < seg; ++k)
            if (b0 + k < a.B) {
                run += s_pref[b0 + k + 1];
                s_pref[b0 + k + 1] = run;
            }
        if (lane == 0) s_pref[0] = 0;
    }
    __syncthreads();
    return s_pref[a.B];
}

__device__ __forceinline__ int bw_find_batch(const int* s_pref, int B, int w) {
    int bl = 0, bh = B;
    while (bh - bl > 1) {
        const int mid = (bl + bh) >> 1;
        if (s_pref[mid] <= w) bl = mid;
        else bh = mid;
    }
    return bl;
}

// Score in log2 units from the raw dot product x: scale, optional soft cap
// (t returned for its derivative), optional ALiBi bias.
template <bool BIAS>
__device__ __forceinline__ float bw_score(const BwdArgs& a, float x, float slope, int dist, float& t) {
    if constexpr (BIAS) {
        float y = x * a.scale;
        t = 0.f;
        if (a.softcap > 0.f) {
            t = fast_tanh(y * (1.f / a.softcap));
            y = a.softcap * t;
        }
        if (a.alibi) y -= slope * (float)(dist < 0 ? -dist : dist);
        return y * kLog2e;
    } else {
        t = 0.f;
        return x * a.scale_log2;
    }
}

// ---- dK, dV ---------------------------------------------------------------------------------
template <int DT, int HD, bool BIAS, bool CHUNK>
__global__ void __launch_bounds__(BwCfg<HD>::KNT, 1) fa_bwd_dkdv_kernel(BwdArgs a) {
    // LDS swizzles for the row length (128-byte rows at head dim 64)
    auto tv = [](int r, int c) { return HD == 64 ? swz_b64(r, c) : swz_v(r, c); };  // row and transpose reads
    auto tk = [](int r, int c) { return HD == 64 ? swz_k64(r, c) : swz_k(r, c); };  // row reads
    using C = BwCfg<HD>;
    constexpr int D = C::D, DCH = C::DCH, KSTEPS = C::KSTEPS, DBLK = C::DBLK, BK = C::BK, BQ = C::BQ,
                  CPQ = C::CPQ, NT = C::KNT, KRB = C::KRB;
    // The q and dout tiles (two buffers each) in one allocation. Head dim 128
    // keeps them as 8-byte halves (split_addr128), and the dout tiles start 8
    // bytes past a 512-byte boundary: no ds_read2 offset can then reach from a
    // q half to a dout half, so the compiler cannot merge a lane's two reads
    // into one ds_read2 (whose two addresses would share banks).
    constexpr bool SPLIT = HD == 128;
    constexpr int QT = BQ * D;                      // elements per tile
    constexpr int DOFF = 2 * QT + (SPLIT ? 4 : 0);  // first dout element
    __shared__ __attribute__((aligned(256))) uint16_t s_qdo[DOFF + 2 * QT];
    auto sq = [&](int buf, int x) -> uint16_t* { return &s_qdo[buf * QT + x]; };
    auto sdo = [&](int buf, int x) -> uint16_t* { return &s_qdo[DOFF + buf * QT + x]; };
    __shared__ __attribute__((aligned(16))) float s_lse[2][BQ];   // lse * log2(e); +inf for rows past the end
    __shared__ __attribute__((aligned(16))) float s_ds[2][BQ];    // dsum
    __shared__ __attribute__((aligned(16))) float s_sl[2][BQ];    // ALiBi slope of the row's head
    __shared__ __attribute__((aligned(16))) int s_pos[2][BQ];     // query position; -1 past the end
    __shared__ int s_pref[bw::kMaxBatch + 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, G = lane >> 4;
    const int total = bw_prefix<NT>(a, s_pref, [&](int b) {
        const BwBatch bb = bw_batch(a, b);
        return a.Hk * ((bb.sk + BK - 1) / BK);
    });

    // LDS offsets: row reads (A operands) and transpose reads, both on the
    // tv layout (head dim 128: the split_addr128 layout of 8-byte halves, row
    // reads as two ds_read_b64, offr[s] the first half, offr[s] ^ 64 the
    // second); staging stores
    int offr[KSTEPS];
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
        offr[s] = SPLIT ? split_addr128(li, G * KSTEPS + s, 0) : li * D + (tv(li, G * KSTEPS + s) << 3);
    const int r4 = li >> 2, c4 = li & 3;
    int offt[DBLK];
#pragma unroll
    for (int db = 0; db < DBLK; ++db)
        offt[db] = SPLIT ? split_addr128(4 * G + r4, 2 * db + (c4 >> 1), c4 & 1)
                         : (4 * G + r4) * D + (tv(4 * G + r4, 2 * db + (c4 >> 1)) << 3) + (c4 & 1) * 4;
    const int dch = tid % DCH, rr0 = tid / DCH;

    const uint16_t* qp = static_cast<const uint16_t*>(a.q);
    const uint16_t* kp = static_cast<const uint16_t*>(a.k);
    const uint16_t* vp = static_cast<const uint16_t*>(a.v);
    const uint16_t* dop = static_cast<const uint16_t*>(a.dout);

    // pass k takes item k * grid + blockIdx.x, the other way round on odd
    // passes (a heavy item of one pass pairs with a light one of the next)
    for (int k = 0; k * (int)gridDim.x < total; ++k) {
        const int w = k * (int)gridDim.x + ((k & 1) ? (int)gridDim.x - 1 - (int)blockIdx.x : (int)blockIdx.x);
        if (w >= total) continue;
        const int b = bw_find_batch(s_pref, a.B, w);
        const BwBatch bb = bw_batch(a, b);
        const int local = w - s_pref[b];
        const int hk = local % a.Hk;
        // heavy first: with only a left window bound, later key blocks see more rows
        const int nkt = (bb.sk + BK - 1) / BK;
        const int kt = (a.wl >= 0 && a.wr < 0) ? nkt - 1 - local / a.Hk : local / a.Hk;
        const int j0 = kt * BK;
        const int g = a.g;
        const UDiv gd = udiv_make((uint32_t)g);  // r / g by a multiply-high in the tile loop
        const int diag0 = bb.sk - bb.sq;
        const int64_t qbase = a.cu_seqlens_q ? (int64_t)a.cu_seqlens_q[b] * a.q_si : (int64_t)b * a.q_sb;
        const int64_t dobase = a.cu_seqlens_q ? (int64_t)a.cu_seqlens_q[b] * a.do_si : (int64_t)b * a.do_sb;
        const int64_t kbase = a.cu_seqlens_k ? (int64_t)a.cu_seqlens_k[b] * a.k_si : (int64_t)b * a.k_sb;
        const int64_t vbase = a.cu_seqlens_k ? (int64_t)a.cu_seqlens_k[b] * a.v_si : (int64_t)b * a.v_sb;

        // this wave's KRB blocks of 16 keys as B operands: block rk, lane holds
        // key (jw + 16*rk + li), chunk G*KSTEPS + s
        const int jw = j0 + 16 * KRB * wave;
        u32x4 kreg[KRB][KSTEPS], vreg[KRB][KSTEPS];
#pragma unroll
        for (int rk = 0; rk < KRB; ++rk) {
            const int jl = jw + 16 * rk + li;
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) {
                const int c = G * KSTEPS + s;
                const bool in = jl < bb.sk && c * 8 < a.hd;
                kreg[rk][s] = in ? *reinterpret_cast<const u32x4*>(kp + kbase + (int64_t)jl * a.k_si + (int64_t)hk * a.k_sh + c * 8)
                                 : u32x4{0u, 0u, 0u, 0u};
                vreg[rk][s] = in ? *reinterpret_cast<const u32x4*>(vp + vbase + (int64_t)jl * a.v_si + (int64_t)hk * a.v_sh + c * 8)
                                 : u32x4{0u, 0u, 0u, 0u};
            }
        }

        // packed rows that can see any key of [j0, j0 + BK)
        int i_lo = 0, i_hi = bb.sq - 1;
        if (a.wr >= 0) i_lo = max(0, j0 - diag0 - a.wr);
        if (a.wl >= 0) i_hi = min(bb.sq - 1, j0 + BK - 1 - diag0 + a.wl);
        if constexpr (CHUNK) {
            i_lo = max(i_lo, row_lo(j0, a.wr, a.chunk) - diag0);
            i_hi = min(i_hi, row_hi(j0 + BK - 1, a.wl, a.chunk) - diag0);
        }
        const int r_lo = i_lo * g;
        const int r_hi = (i_hi >= i_lo) ? (i_hi + 1) * g : r_lo;
        const int ntiles = (r_hi - r_lo + BQ - 1) / BQ;
        // the same range for this wave's keys (skips tiles it cannot see)
        constexpr int WK = 16 * KRB;
        int wi_lo = 0, wi_hi = bb.sq - 1;
        if (a.wr >= 0) wi_lo = max(0, jw - diag0 - a.wr);
        if (a.wl >= 0) wi_hi = min(bb.sq - 1, jw + WK - 1 - diag0 + a.wl);
        const bool wave_live = jw < bb.sk;
        // CHUNK (attention_chunk): rows that see all of the wave's keys,
        // [fc_lo, fc_hi], and the diagonal positions that see this lane's key
        // of block rk, [kc_lo, kc_hi] (window and chunk together)
        [[maybe_unused]] int fc_lo = 0, fc_hi = 0, kc_lo[KRB], kc_hi[KRB];
        if constexpr (CHUNK) {
            wi_lo = max(wi_lo, row_lo(jw, a.wr, a.chunk) - diag0);
            wi_hi = min(wi_hi, row_hi(jw + WK - 1, a.wl, a.chunk) - diag0);
            fc_lo = row_lo(jw + WK - 1, a.wr, a.chunk) - diag0;
            fc_hi = row_hi(jw, a.wl, a.chunk) - diag0;
#pragma unroll
            for (int rk = 0; rk < KRB; ++rk) {
                kc_lo[rk] = row_lo(jw + 16 * rk + li, a.wr, a.chunk);
                kc_hi[rk] = row_hi(jw + 16 * rk + li, a.wl, a.chunk);
            }
        }

        f32x4 dka[KRB][DBLK], dva[KRB][DBLK];
#pragma unroll
        for (int rk = 0; rk < KRB; ++rk)
#pragma unroll
            for (int db = 0; db < DBLK; ++db) {
                dka[rk][db] = f32x4{0.f, 0.f, 0.f, 0.f};
                dva[rk][db] = f32x4{0.f, 0.f, 0.f, 0.f};
            }

        u32x4 qr[CPQ], dr[CPQ];
        float lr = 0.f, dsr = 0.f, slr = 0.f;
        int pr = -1;
        // load_tile is called for the row tiles r_lo, r_lo + BQ, r_lo + 2 BQ, ...
        // in that order. Each thread keeps a cursor per staged row -- the row,
        // its head offset r % g, and its q / dout / lse offsets -- and moves it
        // BQ rows on per call: BQ rows are qB positions and rB heads on, plus
        // one more position when the head offset wraps past g. No products or
        // divisions in the loop (backward 2411-2420 -> 2282-2289 us on the
        // bench shape, same box). The BIAS instances have no registers to spare
        // for the cursors (they would spill 48-76 bytes) and compute each staged
        // row's offsets from its index.
        constexpr bool CURSOR = !BIAS;
        int rnext = r_lo;  // without cursors: the first row of the next tile
        const int qB = (int)udiv(gd, (uint32_t)BQ), rB = BQ - qB * g;
        const int64_t dq0 = (int64_t)qB * a.q_si + (int64_t)rB * a.q_sh, dq1 = dq0 + a.q_si - (int64_t)g * a.q_sh;
        const int64_t dd0 = (int64_t)qB * a.do_si + (int64_t)rB * a.do_sh, dd1 = dd0 + a.do_si - (int64_t)g * a.do_sh;
        const int64_t dl0 = (int64_t)qB + (int64_t)rB * a.lse_sh, dl1 = dl0 + 1 - (int64_t)g * a.lse_sh;
        const uint16_t* qrow = qp + qbase + (int64_t)hk * g * a.q_sh + dch * 8;
        const uint16_t* drow = dop + dobase + (int64_t)hk * g * a.do_sh + dch * 8;
        int cr[CPQ], cj[CPQ];
        int64_t cq[CPQ], cd[CPQ];
        int tr = r_lo + tid, tj = 0, ti = 0;
        int64_t tl = 0;
        if constexpr (CURSOR) {
#pragma unroll
            for (int u = 0; u < CPQ; ++u) {
                cr[u] = r_lo + rr0 + u * (NT / DCH);
                const int i = (int)udiv(gd, (uint32_t)cr[u]);
                cj[u] = cr[u] - i * g;
                cq[u] = (int64_t)i * a.q_si + (int64_t)cj[u] * a.q_sh;
                cd[u] = (int64_t)i * a.do_si + (int64_t)cj[u] * a.do_sh;
            }
            if (tid < BQ) {
                ti = (int)udiv(gd, (uint32_t)tr);
                tj = tr - ti * g;
                tl = (a.cu_seqlens_q ? (int64_t)a.cu_seqlens_q[b] : (int64_t)b * a.lse_sb) +
                     (int64_t)(hk * g + tj) * a.lse_sh + ti;
            }
        }
        auto load_tile = [&]() {
            if constexpr (CURSOR) {
#pragma unroll
                for (int u = 0; u < CPQ; ++u) {
                    if (cr[u] < r_hi && dch * 8 < a.hd) {
                        qr[u] = *reinterpret_cast<const u32x4*>(qrow + cq[u]);
                        dr[u] = *reinterpret_cast<const u32x4*>(drow + cd[u]);
                    } else {
                        qr[u] = u32x4{0u, 0u, 0u, 0u};
                        dr[u] = u32x4{0u, 0u, 0u, 0u};
                    }
                    cr[u] += BQ;
                    cj[u] += rB;
                    const bool wrap = cj[u] >= g;
                    cj[u] = wrap ? cj[u] - g : cj[u];
                    cq[u] += wrap ? dq1 : dq0;
                    cd[u] += wrap ? dd1 : dd0;
                }
                if (tid < BQ) {
                    if (tr < r_hi) {
                        lr = a.lse[tl] * kLog2e;
                        dsr = a.dsum[tl];
                        slr = 0.f;  // no ALiBi without BIAS
                        pr = ti;
                    } else {
                        lr = INFINITY;
                        dsr = 0.f;
                        slr = 0.f;
                        pr = -1;
                    }
                    tr += BQ;
                    ti += qB;
                    tj += rB;
                    const bool wrap = tj >= g;
                    ti = wrap ? ti + 1 : ti;
                    tj = wrap ? tj - g : tj;
                    tl += wrap ? dl1 : dl0;
                }
            } else {
                const int r0 = rnext;
                rnext += BQ;
#pragma unroll
                for (int u = 0; u < CPQ; ++u) {
                    const int r = r0 + rr0 + u * (NT / DCH);
                    if (r < r_hi && dch * 8 < a.hd) {
                        const int i = (int)udiv(gd, (uint32_t)r), j = r - i * g;
                        qr[u] = *reinterpret_cast<const u32x4*>(qrow + (int64_t)i * a.q_si + (int64_t)j * a.q_sh);
                        dr[u] = *reinterpret_cast<const u32x4*>(drow + (int64_t)i * a.do_si + (int64_t)j * a.do_sh);
                    } else {
                        qr[u] = u32x4{0u, 0u, 0u, 0u};
                        dr[u] = u32x4{0u, 0u, 0u, 0u};
                    }
                }
                if (tid < BQ) {
                    const int r = r0 + tid;
                    if (r < r_hi) {
                        const int i = (int)udiv(gd, (uint32_t)r), h = hk * g + (r - i * g);
                        const int64_t lo = a.cu_seqlens_q ? (int64_t)h * a.lse_sh + a.cu_seqlens_q[b] + i
                                                          : (int64_t)b * a.lse_sb + (int64_t)h * a.lse_sh + i;
                        lr = a.lse[lo] * kLog2e;
                        dsr = a.dsum[lo];
                        slr = (BIAS && a.alibi) ? a.alibi[(int64_t)b * a.alibi_sb + h] : 0.f;
                        pr = i;
                    } else {
                        lr = INFINITY;
                        dsr = 0.f;
                        slr = 0.f;
                        pr = -1;
                    }
                }
            }
        };
        auto store_tile = [&](int buf) {
#pragma unroll
            for (int u = 0; u < CPQ; ++u) {
                const int r = rr0 + u * (NT / DCH);
                if constexpr (SPLIT) {
                    const int o0 = split_addr128(r, dch, 0), o1 = o0 ^ 64;
                    *reinterpret_cast<u32x2*>(sq(buf, o0)) = u32x2{qr[u][0], qr[u][1]};
                    *reinterpret_cast<u32x2*>(sq(buf, o1)) = u32x2{qr[u][2], qr[u][3]};
                    *reinterpret_cast<u32x2*>(sdo(buf, o0)) = u32x2{dr[u][0], dr[u][1]};
                    *reinterpret_cast<u32x2*>(sdo(buf, o1)) = u32x2{dr[u][2], dr[u][3]};
                } else {
                    const int off = r * D + (tv(r, dch) << 3);
                    *reinterpret_cast<u32x4*>(sq(buf, off)) = qr[u];
                    *reinterpret_cast<u32x4*>(sdo(buf, off)) = dr[u];
                }
            }
            if (tid < BQ) {
                s_lse[buf][tid] = lr;
                s_ds[buf][tid] = dsr;
                s_sl[buf][tid] = slr;
                s_pos[buf][tid] = pr;
            }
        };

        // 32 rows (half tile hh) against this wave's keys
        auto half = [&](int buf, int hh, auto mask_tag) {
            constexpr bool MASK = decltype(mask_tag)::value;
            f32x4 sacc[KRB][2], pacc[KRB][2];
#pragma unroll
            for (int rk = 0; rk < KRB; ++rk)
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    sacc[rk][t] = f32x4{0.f, 0.f, 0.f, 0.f};
                    pacc[rk][t] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
            // S and dP products at raised wave priority (the SIMD's other
            // wave fills the gaps with its softmax-gradient work): 3172 ->
            // 3111 us for the whole backward of B4 S4096 H32/8 D128 causal,
            // together with the same in the dQ kernel; raising it for the
            // dV/dK products instead is slower (3240 us)
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    u32x4 aq, ad;
                    if constexpr (SPLIT) {
                        // LDS byte address of the first half; opaque to the
                        // compiler, since reads 16 rows apart would otherwise
                        // merge into ds_read2st64_b64, which reads both of a
                        // lane's addresses (same banks) in one pass. The second
                        // half is the other 128-byte plane (256-byte aligned
                        // rows), the dout tile a fixed distance away.
                        unsigned a0 = lds_addr(sq(buf, offr[s] + t * 16 * D));
                        asm volatile("" : "+v"(a0));
                        const unsigned a1 = a0 ^ 128u;
                        constexpr unsigned DO = 2 * DOFF;  // bytes from a q element to its dout element
                        const u32x2 q0 = lds_load_u32x2(a0 + hh * 32 * D * 2);
                        const u32x2 q1 = lds_load_u32x2(a1 + hh * 32 * D * 2);
                        const u32x2 d0 = lds_load_u32x2(a0 + DO + hh * 32 * D * 2);
                        const u32x2 d1 = lds_load_u32x2(a1 + DO + hh * 32 * D * 2);
                        aq = u32x4{q0[0], q0[1], q1[0], q1[1]};
                        ad = u32x4{d0[0], d0[1], d1[0], d1[1]};
                    } else {
                        const int ro = (hh * 32 + t * 16) * D + offr[s];
                        aq = *reinterpret_cast<const u32x4*>(sq(buf, ro));
                        ad = *reinterpret_cast<const u32x4*>(sdo(buf, ro));
                    }
#pragma unroll
                    for (int rk = 0; rk < KRB; ++rk) {
                        sacc[rk][t] = mfma16x16x32<DT>(aq, kreg[rk][s], sacc[rk][t]);
                        pacc[rk][t] = mfma16x16x32<DT>(ad, vreg[rk][s], pacc[rk][t]);
                    }
                }
            }
            __builtin_amdgcn_s_setprio(0);
            // lane: key jw + 16rk + li, rows hh*32 + 16t + 4G + e
            f32x4 l4[2], d4[2];
            [[maybe_unused]] f32x4 sl4[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
            [[maybe_unused]] int p4[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int ro = hh * 32 + t * 16 + 4 * G;
                l4[t] = *reinterpret_cast<const f32x4*>(&s_lse[buf][ro]);
                d4[t] = *reinterpret_cast<const f32x4*>(&s_ds[buf][ro]);
                if constexpr (BIAS) sl4[t] = *reinterpret_cast<const f32x4*>(&s_sl[buf][ro]);
                if constexpr (MASK || BIAS) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) p4[t][e] = s_pos[buf][ro + e];
                }
            }
            u32x4 pk[KRB], dk[KRB];
#pragma unroll
            for (int rk = 0; rk < KRB; ++rk) {
                const int jl = jw + 16 * rk + li;
                float p[2][4], ds[2][4];
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float th;
                        const float x = bw_score<BIAS>(a, sacc[rk][t][e], sl4[t][e], p4[t][e] + diag0 - jl, th);
                        float pv = fast_exp2(x - l4[t][e]);
                        if constexpr (MASK) {
                            const int dg = p4[t][e] + diag0;
                            bool vis = p4[t][e] >= 0 && jl < bb.sk;
                            if constexpr (CHUNK) {
                                vis = vis && dg >= kc_lo[rk] && dg <= kc_hi[rk];
                            } else {
                                if (a.wl >= 0 && jl < dg - a.wl) vis = false;
                                if (a.wr >= 0 && jl > dg + a.wr) vis = false;
                            }
                            pv = vis ? pv : 0.f;
                        }
                        // dS without the softmax scale, which is applied to dK once at the end
                        float dsv = pv * (pacc[rk][t][e] - d4[t][e]);
                        if constexpr (BIAS) dsv *= 1.f - th * th;
                        p[t][e] = pv;
                        ds[t][e] = dsv;
                    }
                pk[rk] = pack8<DT>(f32x8{p[0][0], p[0][1], p[0][2], p[0][3], p[1][0], p[1][1], p[1][2], p[1][3]});
                dk[rk] = pack8<DT>(f32x8{ds[0][0], ds[0][1], ds[0][2], ds[0][3], ds[1][0], ds[1][1], ds[1][2], ds[1][3]});
            }
            // dV^T += dO^T . P and dK^T += Q^T . dS (transpose reads of the
            // tiles, shared by the wave's key blocks)
#pragma unroll
            for (int db = 0; db < DBLK; ++db) {
                const int o0 = offt[db] + (32 * hh) * D, o1 = offt[db] + (32 * hh + 16) * D;
                const u32x2 dl = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)sdo(buf, o0)));
                const u32x2 dh = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)sdo(buf, o1)));
                const u32x2 ql = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)sq(buf, o0)));
                const u32x2 qh = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)sq(buf, o1)));
                const u32x4 dot = {dl[0], dl[1], dh[0], dh[1]}, qt = {ql[0], ql[1], qh[0], qh[1]};
#pragma unroll
                for (int rk = 0; rk < KRB; ++rk) {
                    dva[rk][db] = mfma16x16x32<DT>(dot, pk[rk], dva[rk][db]);
                    dka[rk][db] = mfma16x16x32<DT>(qt, dk[rk], dka[rk][db]);
                }
            }
        };

        if (ntiles > 0) {
            load_tile();
            store_tile(0);
            if (ntiles > 1) load_tile();
        }
        __syncthreads();
        for (int t = 0; t < ntiles; ++t) {
            const int buf = t & 1;
            const int rt = r_lo + t * BQ;
            if (wave_live) {
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int h0 = rt + 32 * hh;  // first packed row of the half
                    if (h0 >= r_hi) continue;
                    const int p_lo = (int)udiv(gd, (uint32_t)h0), p_hi = (int)udiv(gd, (uint32_t)min(h0 + 31, r_hi - 1));
                    if (p_hi < wi_lo || p_lo > wi_hi) continue;  // no row of the half sees these keys
                    bool full = h0 + 32 <= r_hi && jw + WK <= bb.sk;
                    if (a.wr >= 0 && jw + WK - 1 > p_lo + diag0 + a.wr) full = false;
                    if (a.wl >= 0 && jw < p_hi + diag0 - a.wl) full = false;
                    if constexpr (CHUNK) {
                        if (p_lo < fc_lo || p_hi > fc_hi) full = false;
                    }
                    if (full) half(buf, hh, std::integral_constant<bool, false>{});
                    else half(buf, hh, std::integral_constant<bool, true>{});
                }
            }
            if (t + 1 < ntiles) store_tile(buf ^ 1);
            if (t + 2 < ntiles) load_tile();
            __syncthreads();
        }

        // lane holds dK^T / dV^T [dims 16db + 4G + i][key jw + 16rk + li]
        if (wave_live) {
#pragma unroll
            for (int rk = 0; rk < KRB; ++rk) {
                const int jl = jw + 16 * rk + li;
                if (jl >= bb.sk) continue;
                uint16_t* dkp = static_cast<uint16_t*>(a.dk) +
                                (a.cu_seqlens_k ? (int64_t)a.cu_seqlens_k[b] * a.dk_si : (int64_t)b * a.dk_sb) +
                                (int64_t)jl * a.dk_si + (int64_t)hk * a.dk_sh;
                uint16_t* dvp = static_cast<uint16_t*>(a.dv) +
                                (a.cu_seqlens_k ? (int64_t)a.cu_seqlens_k[b] * a.dv_si : (int64_t)b * a.dv_sb) +
                                (int64_t)jl * a.dv_si + (int64_t)hk * a.dv_sh;
#pragma unroll
                for (int db = 0; db < DBLK; ++db) {
                    if (16 * db + 4 * G >= a.hd) continue;
                    const f32x4 kk = dka[rk][db] * a.scale;
                    uint16_t k4[4] = {f32_to_16<DT>(kk[0]), f32_to_16<DT>(kk[1]), f32_to_16<DT>(kk[2]), f32_to_16<DT>(kk[3])};
                    uint16_t v4[4] = {f32_to_16<DT>(dva[rk][db][0]), f32_to_16<DT>(dva[rk][db][1]),
                                      f32_to_16<DT>(dva[rk][db][2]), f32_to_16<DT>(dva[rk][db][3])};
                    *reinterpret_cast<u32x2*>(dkp + 16 * db + 4 * G) = __builtin_bit_cast(u32x2, k4);
                    *reinterpret_cast<u32x2*>(dvp + 16 * db + 4 * G) = __builtin_bit_cast(u32x2, v4);
                }
            }
        }
    }
}

// ---- dQ -------------------------------------------------------------------------------------
template <int DT, int HD, bool BIAS>
__global__ void __launch_bounds__(BwCfg<HD>::QNT, 1) fa_bwd_dq_kernel(BwdArgs a) {
    // LDS swizzles for the row length (128-byte rows at head dim 64)
    auto tv = [](int r, int c) { return HD == 64 ? swz_b64(r, c) : swz_v(r, c); };  // row and transpose reads
    auto tk = [](int r, int c) { return HD == 64 ? swz_k64(r, c) : swz_k(r, c); };  // row reads
    using C = BwCfg<HD>;
    constexpr int D = C::D, DCH = C::DCH, KSTEPS = C::KSTEPS, DBLK = C::DBLK, RB = C::RB, BM = C::BM, BN = C::BN,
                  CPK = C::CPK, NT = C::QNT;
    // K tiles (tv: row reads and transpose reads) and V tiles (tk: row reads),
    // two buffers each, in one allocation. Head dim 128 keeps both as 8-byte
    // halves (split_addr128) and starts the V tiles 8 bytes past a 512-byte
    // boundary, so a lane's K and V reads cannot merge into one ds_read2
    // (whose two addresses would share banks).
    constexpr bool SPLIT = HD == 128;
    constexpr int KT = BN * D;                      // elements per tile
    constexpr int VOFF = 2 * KT + (SPLIT ? 4 : 0);  // first V element
    __shared__ __attribute__((aligned(256))) uint16_t s_kv[VOFF + 2 * KT];
    auto sk = [&](int buf, int x) -> uint16_t* { return &s_kv[buf * KT + x]; };
    auto sv = [&](int buf, int x) -> uint16_t* { return &s_kv[VOFF + buf * KT + x]; };
    __shared__ int s_pref[bw::kMaxBatch + 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, G = lane >> 4;
    const int total = bw_prefix<NT>(a, s_pref, [&](int b) {
        const BwBatch bb = bw_batch(a, b);
        return a.Hk * ((bb.rows + BM - 1) / BM);
    });

    // row-read offsets of K and V (head dim 128: the first 8-byte half, the
    // same for both tiles; the second half is ^ 64) and K^T transpose reads
    int offkr[KSTEPS], offvr[SPLIT ? 1 : KSTEPS];
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
        if constexpr (SPLIT) {
            offkr[s] = split_addr128(li, G * KSTEPS + s, 0);
        } else {
            offkr[s] = li * D + (tv(li, G * KSTEPS + s) << 3);
            offvr[s] = li * D + (tk(li, G * KSTEPS + s) << 3);
        }
    }
    const int r4 = li >> 2, c4 = li & 3;
    int offt[DBLK];
#pragma unroll
    for (int db = 0; db < DBLK; ++db)
        offt[db] = SPLIT ? split_addr128(4 * G + r4, 2 * db + (c4 >> 1), c4 & 1)
                         : (4 * G + r4) * D + (tv(4 * G + r4, 2 * db + (c4 >> 1)) << 3) + (c4 & 1) * 4;
    const int dch = tid % DCH, kk0 = tid / DCH;

    const uint16_t* qp = static_cast<const uint16_t*>(a.q);
    const uint16_t* kp = static_cast<const uint16_t*>(a.k);
    const uint16_t* vp = static_cast<const uint16_t*>(a.v);
    const uint16_t* dop = static_cast<const uint16_t*>(a.dout);
    const uint16_t* outp = static_cast<const uint16_t*>(a.out);

    // pass k takes item k * grid + blockIdx.x, the other way round on odd
    // passes (a heavy item of one pass pairs with a light one of the next)
    for (int k = 0; k * (int)gridDim.x < total; ++k) {
        const int w = k * (int)gridDim.x + ((k & 1) ? (int)gridDim.x - 1 - (int)blockIdx.x : (int)blockIdx.x);
        if (w >= total) continue;
        const int b = bw_find_batch(s_pref, a.B, w);
        const BwBatch bb = bw_batch(a, b);
        const int local = w - s_pref[b];
        const int hk = local % a.Hk;
        // heavy first: with a right window bound (causal), later row tiles see
        // more keys, and the hardware dispatches the workgroups in order
        const int nmt = (bb.rows + BM - 1) / BM;
        const int mt = a.wr >= 0 ? nmt - 1 - local / a.Hk : local / a.Hk;
        const int g = a.g;
        const int diag0 = bb.sk - bb.sq;
        const int tile_row0 = mt * BM;
        const int tile_rows = min(BM, bb.rows - tile_row0);
        int k_lo = 0, k_hi = bb.sk;
        {
            const int i_lo = tile_row0 / g, i_hi = (tile_row0 + tile_rows - 1) / g;
            k_lo = max(0, key_lo(i_lo + diag0, a.wl, a.chunk));
            k_hi = min(bb.sk, key_hi(i_hi + diag0, a.wr, a.chunk) + 1);
            if (k_hi < k_lo) k_hi = k_lo;
        }
        const int ntiles = (k_hi - k_lo + BN - 1) / BN;
        const int wrow0 = tile_row0 + wave * RB * 16;
        const int wrows = min(RB * 16, bb.rows - wrow0);
        const bool wave_live = wrows > 0;
        const int wi_lo = wave_live ? wrow0 / g : 0;
        const int wi_hi = wave_live ? (wrow0 + wrows - 1) / g : 0;
        // keys visible to some row of the wave: [w_lo, w_hi]; to every row: [f_lo, f_hi]
        const int w_lo = key_lo(wi_lo + diag0, a.wl, a.chunk), w_hi = key_hi(wi_hi + diag0, a.wr, a.chunk);
        const int f_lo = key_lo(wi_hi + diag0, a.wl, a.chunk), f_hi = key_hi(wi_lo + diag0, a.wr, a.chunk);

        const int64_t qbase = a.cu_seqlens_q ? (int64_t)a.cu_seqlens_q[b] * a.q_si : (int64_t)b * a.q_sb;
        const int64_t dobase = a.cu_seqlens_q ? (int64_t)a.cu_seqlens_q[b] * a.do_si : (int64_t)b * a.do_sb;
        const int64_t kbase = a.cu_seqlens_k ? (int64_t)a.cu_seqlens_k[b] * a.k_si : (int64_t)b * a.k_sb;
        const int64_t vbase = a.cu_seqlens_k ? (int64_t)a.cu_seqlens_k[b] * a.v_si : (int64_t)b * a.v_sb;

        // q and dout rows as B operands; lse (log2 units) per row; dsum per row
        // from the out rows and the dout rows loaded here (this kernel runs
        // first and writes dsum for the dK/dV kernel and softmax_d)
        const int64_t obase = a.cu_seqlens_q ? (int64_t)a.cu_seqlens_q[b] * a.o_si : (int64_t)b * a.o_sb;
        u32x4 qreg[RB][KSTEPS], dreg[RB][KSTEPS], oreg[RB][KSTEPS];
        float lse2[RB], dsv[RB], slope[RB];
        int64_t lor[RB];
        int qi[RB], rlo[RB], rhi[RB];  // rlo/rhi: the row's visible keys before the clamp to k_hi
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int r = wrow0 + rb * 16 + li;
            const bool ok = r < bb.rows;
            const int i = ok ? r / g : 0;
            const int h = hk * g + (ok ? r % g : 0);
            qi[rb] = i;
            rlo[rb] = key_lo(i + diag0, a.wl, a.chunk);
            rhi[rb] = key_hi(i + diag0, a.wr, a.chunk);
            const int64_t lo = a.cu_seqlens_q ? (int64_t)h * a.lse_sh + a.cu_seqlens_q[b] + i
                                              : (int64_t)b * a.lse_sb + (int64_t)h * a.lse_sh + i;
            lse2[rb] = ok ? a.lse[lo] * kLog2e : INFINITY;
            lor[rb] = ok ? lo : -1;
            slope[rb] = (BIAS && a.alibi && ok) ? a.alibi[(int64_t)b * a.alibi_sb + h] : 0.f;
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) {
                const int c = G * KSTEPS + s;
                const bool in = ok && c * 8 < a.hd;
                qreg[rb][s] = in ? *reinterpret_cast<const u32x4*>(qp + qbase + (int64_t)i * a.q_si + (int64_t)h * a.q_sh + c * 8)
                                 : u32x4{0u, 0u, 0u, 0u};
                dreg[rb][s] = in ? *reinterpret_cast<const u32x4*>(dop + dobase + (int64_t)i * a.do_si + (int64_t)h * a.do_sh + c * 8)
                                 : u32x4{0u, 0u, 0u, 0u};
                oreg[rb][s] = in ? *reinterpret_cast<const u32x4*>(outp + obase + (int64_t)i * a.o_si + (int64_t)h * a.o_sh + c * 8)
                                 : u32x4{0u, 0u, 0u, 0u};
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): retire the row loads before the tile loop
        // dsum = rowsum(dout * out): the 4 lanes li, li + 16, li + 32, li + 48 hold a row's dims
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            float acc = 0.f;
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) {
                uint16_t oh[8], dh[8];
                __builtin_memcpy(oh, &oreg[rb][s], 16);
                __builtin_memcpy(dh, &dreg[rb][s], 16);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc += f16_to_32<DT>(oh[e]) * f16_to_32<DT>(dh[e]);
            }
            acc += __shfl_xor(acc, 16);
            acc += __shfl_xor(acc, 32);
            dsv[rb] = lor[rb] >= 0 ? acc : 0.f;
            if (G == 0 && lor[rb] >= 0) a.dsum[lor[rb]] = acc;
        }

        f32x4 dqa[RB][DBLK];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int db = 0; db < DBLK; ++db) dqa[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};

        u32x4 kr[CPK], vr[CPK];
        auto load_tile = [&](int t0) {
#pragma unroll
            for (int u = 0; u < CPK; ++u) {
                const int j = t0 + kk0 + u * (NT / DCH);
                if (j < k_hi && dch * 8 < a.hd) {
                    kr[u] = *reinterpret_cast<const u32x4*>(kp + kbase + (int64_t)j * a.k_si + (int64_t)hk * a.k_sh + dch * 8);
                    vr[u] = *reinterpret_cast<const u32x4*>(vp + vbase + (int64_t)j * a.v_si + (int64_t)hk * a.v_sh + dch * 8);
                } else {
                    kr[u] = u32x4{0u, 0u, 0u, 0u};
                    vr[u] = u32x4{0u, 0u, 0u, 0u};
                }
            }
        };
        auto store_tile = [&](int buf) {
#pragma unroll
            for (int u = 0; u < CPK; ++u) {
                const int r = kk0 + u * (NT / DCH);
                if constexpr (SPLIT) {
                    const int o0 = split_addr128(r, dch, 0), o1 = o0 ^ 64;
                    *reinterpret_cast<u32x2*>(sk(buf, o0)) = u32x2{kr[u][0], kr[u][1]};
                    *reinterpret_cast<u32x2*>(sk(buf, o1)) = u32x2{kr[u][2], kr[u][3]};
                    *reinterpret_cast<u32x2*>(sv(buf, o0)) = u32x2{vr[u][0], vr[u][1]};
                    *reinterpret_cast<u32x2*>(sv(buf, o1)) = u32x2{vr[u][2], vr[u][3]};
                } else {
                    *reinterpret_cast<u32x4*>(sk(buf, r * D + (tv(r, dch) << 3))) = kr[u];
                    *reinterpret_cast<u32x4*>(sv(buf, r * D + (tk(r, dch) << 3))) = vr[u];
                }
            }
        };

        // 32 keys (half hh of the LDS tile) for this wave's rows
        auto half = [&](int buf, int hh, int s0, auto mask_tag) {
            constexpr bool MASK = decltype(mask_tag)::value;
            f32x4 sacc[RB][2], pacc[RB][2];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    sacc[rb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
                    pacc[rb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
            // S^T and dP^T products at raised wave priority (see the dK/dV kernel)
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    u32x4 ak, av;
                    if constexpr (SPLIT) {
                        // opaque LDS byte address of the first half (reads 16
                        // rows apart would merge into ds_read2st64_b64, which
                        // reads both of a lane's addresses in one pass)
                        unsigned a0 = lds_addr(sk(buf, offkr[s] + kb * 16 * D));
                        asm volatile("" : "+v"(a0));
                        const unsigned a1 = a0 ^ 128u;
                        constexpr unsigned VO = 2 * VOFF;  // bytes from a K element to its V element
                        const u32x2 k0 = lds_load_u32x2(a0 + hh * 32 * D * 2);
                        const u32x2 k1 = lds_load_u32x2(a1 + hh * 32 * D * 2);
                        const u32x2 v0 = lds_load_u32x2(a0 + VO + hh * 32 * D * 2);
                        const u32x2 v1 = lds_load_u32x2(a1 + VO + hh * 32 * D * 2);
                        ak = u32x4{k0[0], k0[1], k1[0], k1[1]};
                        av = u32x4{v0[0], v0[1], v1[0], v1[1]};
                    } else {
                        ak = *reinterpret_cast<const u32x4*>(sk(buf, offkr[s] + (hh * 32 + kb * 16) * D));
                        av = *reinterpret_cast<const u32x4*>(sv(buf, offvr[s] + (hh * 32 + kb * 16) * D));
                    }
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) {
                        sacc[rb][kb] = mfma16x16x32<DT>(ak, qreg[rb][s], sacc[rb][kb]);
                        pacc[rb][kb] = mfma16x16x32<DT>(av, dreg[rb][s], pacc[rb][kb]);
                    }
                }
            }
            __builtin_amdgcn_s_setprio(0);
            // lane: row li of block rb, keys s0 + 16kb + 4G + e
            u32x4 dsk[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                float ds[2][4];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int j = s0 + kb * 16 + 4 * G + e;
                        float th;
                        const float x = bw_score<BIAS>(a, sacc[rb][kb][e], slope[rb], qi[rb] + diag0 - j, th);
                        float pv = fast_exp2(x - lse2[rb]);
                        if constexpr (MASK) {
                            const bool vis = j < k_hi && j >= rlo[rb] && j <= rhi[rb];
                            pv = vis ? pv : 0.f;
                        }
                        // dS without the softmax scale, which is applied to dQ once at the end
                        float d = pv * (pacc[rb][kb][e] - dsv[rb]);
                        if constexpr (BIAS) d *= 1.f - th * th;
                        ds[kb][e] = d;
                    }
                dsk[rb] = pack8<DT>(f32x8{ds[0][0], ds[0][1], ds[0][2], ds[0][3], ds[1][0], ds[1][1], ds[1][2], ds[1][3]});
            }
            // dQ^T += K^T . dS^T
#pragma unroll
            for (int db = 0; db < DBLK; ++db) {
                const u32x2 l2 = __builtin_bit_cast(
                    u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)sk(buf, offt[db] + (32 * hh) * D)));
                const u32x2 h2 = __builtin_bit_cast(
                    u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)sk(buf, offt[db] + (32 * hh + 16) * D)));
                const u32x4 kt = {l2[0], l2[1], h2[0], h2[1]};
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) dqa[rb][db] = mfma16x16x32<DT>(kt, dsk[rb], dqa[rb][db]);
            }
        };

        if (ntiles > 0) {
            load_tile(k_lo);
            store_tile(0);
            if (ntiles > 1) load_tile(k_lo + BN);
        }
        __syncthreads();
        for (int t = 0; t < ntiles; ++t) {
            const int buf = t & 1;
            const int s0 = k_lo + t * BN, s1 = s0 + BN;
            const bool skip = !wave_live || s0 > w_hi || s1 - 1 < w_lo;
            if (!skip) {
#pragma unroll
                for (int hh = 0; hh < BN / 32; ++hh) {
                    const int h0 = s0 + 32 * hh, h1 = h0 + 32;
                    if (h0 >= k_hi || h0 > w_hi || h1 - 1 < w_lo) continue;
                    const bool full = h1 <= k_hi && h0 >= f_lo && h1 - 1 <= f_hi;
                    if (full) half(buf, hh, h0, std::integral_constant<bool, false>{});
                    else half(buf, hh, h0, std::integral_constant<bool, true>{});
                }
            }
            if (t + 1 < ntiles) store_tile(buf ^ 1);
            if (t + 2 < ntiles) load_tile(k_lo + (t + 2) * BN);
            __syncthreads();
        }

        // lane holds dQ^T [dims 16db + 4G + i][row li of block rb]
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int r = wrow0 + rb * 16 + li;
            if (r >= bb.rows) continue;
            const int i = r / g, h = hk * g + r % g;
            uint16_t* row = static_cast<uint16_t*>(a.dq) +
                            (a.cu_seqlens_q ? (int64_t)a.cu_seqlens_q[b] * a.dq_si : (int64_t)b * a.dq_sb) +
                            (int64_t)i * a.dq_si + (int64_t)h * a.dq_sh;
#pragma unroll
            for (int db = 0; db < DBLK; ++db) {
                if (16 * db + 4 * G >= a.hd) continue;
                const f32x4 qq = dqa[rb][db] * a.scale;
                uint16_t q4[4] = {f32_to_16<DT>(qq[0]), f32_to_16<DT>(qq[1]), f32_to_16<DT>(qq[2]), f32_to_16<DT>(qq[3])};
                *reinterpret_cast<u32x2*>(row + 16 * db + 4 * G) = __builtin_bit_cast(u32x2, q4);
            }
        }
    }
}

// ---- host-side launchers (called from fa_api.cpp) -------------------------------------------
// attention_chunk runs the dK/dV kernel's CHUNK instance (on the general score
// path); the common instances keep the plain window masks, whose code the
// chunk tests would slow down.
template <int DT, int HD, bool BIAS>
static void launch_bwd_t(const BwdArgs& a, int grid_kv, int grid_q, hipStream_t stream) {
    hipLaunchKernelGGL((fa_bwd_dq_kernel<DT, HD, BIAS>), dim3(grid_q), dim3(BwCfg<HD>::QNT), 0, stream, a);
    if (a.chunk > 0)
        hipLaunchKernelGGL((fa_bwd_dkdv_kernel<DT, HD, true, true>), dim3(grid_kv), dim3(BwCfg<HD>::KNT), 0, stream, a);
    else
        hipLaunchKernelGGL((fa_bwd_dkdv_kernel<DT, HD, BIAS, false>), dim3(grid_kv), dim3(BwCfg<HD>::KNT), 0, stream, a);
}

template <int HD>
static void launch_bwd_d(const BwdArgs& a, int dtype, int grid_kv, int grid_q, hipStream_t stream) {
    const bool bias = a.softcap > 0.f || a.alibi != nullptr || !(a.scale > 0.f);
    if (dtype == DT_BF16) {
        if (bias) launch_bwd_t<DT_BF16, HD, true>(a, grid_kv, grid_q, stream);
        else launch_bwd_t<DT_BF16, HD, false>(a, grid_kv, grid_q, stream);
    } else {
        if (bias) launch_bwd_t<DT_FP16, HD, true>(a, grid_kv, grid_q, stream);
        else launch_bwd_t<DT_FP16, HD, false>(a, grid_kv, grid_q, stream);
    }
}

int bwd_key_block(int d) { return d > 128 ? BwCfg<256>::BK : d > 64 ? BwCfg<128>::BK : BwCfg<64>::BK; }
int bwd_row_block(int d) { return d > 128 ? BwCfg<256>::BM : d > 64 ? BwCfg<128>::BM : BwCfg<64>::BM; }

// d: kernel head dim (128 or 256); grids: upper bounds on the work items of each kernel
hipError_t launch_bwd(const BwdArgs& a, int dtype, int d, int grid_kv, int grid_q, hipStream_t stream) {
    if (d != 64 && d != 128 && d != 256) return hipErrorInvalidValue;
    if (d == 64) launch_bwd_d<64>(a, dtype, grid_kv, grid_q, stream);
    else if (d == 128) launch_bwd_d<128>(a, dtype, grid_kv, grid_q, stream);
    else launch_bwd_d<256>(a, dtype, grid_kv, grid_q, stream);
    return hipGetLastError();
}

}  // namespace fa
