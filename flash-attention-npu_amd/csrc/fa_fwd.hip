// fa_fwd.hip -- FlashAttention forward (prefill / chunked prefill / dense /
// varlen) for gfx950 (MI355X), the split-KV merge, and the standalone
// log-sum-exp combine.
//
// Reference behaviour being reproduced (paths relative to the reference repo):
//   SplitFuse::FAInfer / runMainLoop  csrc/arch22/flash_attn_npu_v2/mha_fwd_kvcache.cpp:436-966
//   online softmax                    csrc/arch22/flash_attn_npu_v2/online_softmax.hpp:477-803
//   rescale / finalize / LSE          csrc/arch22/flash_attn_npu_v2/rescale_o.hpp:299-534
//   split-KV combine                  csrc/arch22/flash_attn_npu_v2/CombineScale.hpp:76-357
//   split planner                     csrc/arch22/flash_attn_npu_v3/fa_split.h:483-510
// The design is MI355X-native rather than a translation:
//   * Rows of a work tile are (query position, q head) pairs of ONE kv head
//     (GQA packing: row r -> position r / g, head hk*g + r % g), so each K/V
//     byte fetched from HBM serves all g query heads.
//   * S^T = K.Q^T with 16x16x32 MFMA: the accumulator then holds, per lane, one
//     query row and 8 keys, which is exactly the packed P^T operand of
//     O^T = V^T.P^T. The head dimension of Q/K is permuted (lane group G takes
//     dims G*D/4 .. +D/4) so every lane reads contiguous 16-byte chunks.
//   * One workgroup = 8 waves x 32 rows (two waves per SIMD); a wave reuses
//     each K/V operand it reads from LDS for its 2 row blocks of 16. The
//     256-VGPR budget of two waves per SIMD is what bounds the row blocks.
//   * With kvcache rotary, q is rotated as it is loaded (ROT), so the rotated
//     copy is never written to or re-read from HBM.
//   * K/V tiles (64 keys) are double-buffered in LDS with one barrier per
//     tile; K uses a 16-byte XOR swizzle on the row, V one on the low row bits
//     so that both the K operand reads and the ds_read_b64_tr_b16 transpose
//     reads of V^T are bank-conflict free.
//   * Online softmax in fp32 in the log2 domain with a lazy maximum: the
//     running max moves (and O, l are rescaled) only when a row's new scores
//     exceed it by more than 2^8, so the common path has no cross-lane
//     reduction and no O rescale. P is rounded to the input dtype before P.V,
//     the row sum uses the fp32 P (tests/test_flash_attn_npu_v3.py:29-47,130).
//   * Masks are evaluated per tile: fully visible tiles skip the per-element
//     test and fully hidden tiles are skipped.
//   * The split plan (for few, long sequences) is made by every workgroup from
//     the sequence lengths in LDS; there is no host round trip.
#include "fa_common.h"
#include "fa_kernel_args.h"
#include "fa_rope.h"

#include <type_traits>

namespace fa {

constexpr int kMaxBatchLds = 2048;

struct BatchInfo {
    int sq, sk, rows, mt, lo, hi;
    int len0;  // kvcache: cache_seqlens[b] before this call's append, else 0
    int lp;    // kvcache: cache_leftpad[b] (key j is cache row lp + j), else 0
};

template <int BM>
__device__ __forceinline__ void batch_info(const FwdArgs& a, int b, BatchInfo& bi) {
    int sq = a.cu_seqlens_q ? a.cu_seqlens_q[b + 1] - a.cu_seqlens_q[b] : a.Sq;
    int sk;
    bi.len0 = a.seqlens_k ? a.seqlens_k[b] : 0;
    bi.lp = a.leftpad ? min(max(a.leftpad[b], 0), a.kv_capacity) : 0;
    if (a.seqlens_k)  // cache_seqlens (+ this call's new tokens) / seqused_k
        sk = bi.len0 + (a.cu_knew ? a.cu_knew[b + 1] - a.cu_knew[b] : a.seqlen_new) - bi.lp;
    else if (a.cu_seqlens_k) sk = a.cu_seqlens_k[b + 1] - a.cu_seqlens_k[b];
    else sk = a.Sk;
    sq = min(max(sq, 0), a.Sq);  // Sq is max_seqlen_q for varlen: bounds the tiles
    sk = min(max(sk, 0), a.kv_capacity - bi.lp);
    bi.sq = sq;
    bi.sk = sk;
    bi.rows = sq * a.g;
    bi.mt = (bi.rows + BM - 1) / BM;
    // union of the keys visible to any row of this sequence
    const int lo = max(0, key_lo(sk - sq, a.wl, a.chunk));
    const int hi = min(sk, key_hi(sk - 1, a.wr, a.chunk) + 1);
    bi.lo = lo;
    bi.hi = max(hi, lo);
}

__device__ __forceinline__ void split_of(const FwdArgs& a, int range, int chunk_auto, int& ns, int& chunk) {
    if (!a.allow_split || range <= 0) {
        ns = 1;
        chunk = max(range, 1);
    } else if (a.num_splits > 0) {
        ns = a.num_splits;
        chunk = (range + ns - 1) / ns;
    } else {
        chunk = chunk_auto;
        ns = (range + chunk - 1) / chunk;
    }
}

// Builds the per-batch work prefix in LDS. Every workgroup computes the same
// plan; workgroup 0 also publishes it for the combine kernel.
template <int BM, int BN, int NT, int NW>
__device__ void build_schedule(const FwdArgs& a, int* s_pref, long long* s_red, int& total, int& chunk_auto) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    long long work = 0, base = 0;
    for (int b = tid; b < a.B; b += NT) {
        BatchInfo bi;
        batch_info<BM>(a, b, bi);
        long long tiles = (long long)a.Hk * bi.mt;
        base += tiles;
        work += tiles * (bi.hi - bi.lo);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        work += __shfl_xor(work, o);
        base += __shfl_xor(base, o);
    }
    if (lane == 0) {
        s_red[wave * 2] = work;
        s_red[wave * 2 + 1] = base;
    }
    __syncthreads();
    work = 0;
    base = 0;
    for (int w = 0; w < NW; ++w) {
        work += s_red[w * 2];
        base += s_red[w * 2 + 1];
    }
    int ca = 0x3fffffff;
    if (a.allow_split && a.num_splits <= 0 && base < a.target_items) {
        long long c = (work + a.target_items - 1) / a.target_items;
        c = c < a.min_chunk ? a.min_chunk : c;
        c = (c + BN - 1) / BN * BN;
        ca = (int)(c > 0x3fffffff ? 0x3fffffff : c);
    }
    chunk_auto = ca;
    for (int b = tid; b < a.B; b += NT) {
        BatchInfo bi;
        batch_info<BM>(a, b, bi);
        int ns, chunk;
        split_of(a, bi.hi - bi.lo, ca, ns, chunk);
        s_pref[b + 1] = a.Hk * bi.mt * ns;
        if (blockIdx.x == 0 && a.sched) a.sched[a.B + 1 + b] = ns;
    }
    __syncthreads();
    if (wave == 0) {
        const int seg = (a.B + 63) / 64;
        const int b0 = lane * seg;
        int local = 0;
        for (int k = 0; k < seg; ++k) {
            int b = b0 + k;
            if (b < a.B) local += s_pref[b + 1];
        }
        int incl = local;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            int v = __shfl_up(incl, o);
            if (lane >= o) incl += v;
        }
        int run = incl - local;
        for (int k = 0; k < seg; ++k) {
            int b = b0 + k;
            if (b < a.B) {
                run += s_pref[b + 1];
                s_pref[b + 1] = run;
            }
        }
        if (lane == 0) s_pref[0] = 0;
    }
    __syncthreads();
    total = s_pref[a.B];
    if (blockIdx.x == 0 && a.sched) {
        for (int b = tid; b <= a.B; b += NT) a.sched[b] = s_pref[b];
    }
}





namespace pf {
constexpr float kLazy = 8.f;       // log2 headroom before the running max moves
}  // namespace pf

// Tile shape per kernel head dim (128 or 256; smaller head dims run on the
// 128 kernel with the dims above them read as zero). At 256 a wave keeps one
// 16-row block: its q operands and O accumulators take twice the registers.
template <int HD>
struct PfCfg {
    static constexpr int D = HD;
    static constexpr int RB = HD > 128 ? 1 : HD == 64 ? 4 : 2;  // 16-row blocks per wave
    static constexpr int NW = 8;                      // waves per workgroup
    static constexpr int NT = NW * 64;
    static constexpr int BM = NW * RB * 16;           // packed rows per work tile
    static constexpr int BN = HD > 128 ? 32 : 64;     // keys per LDS tile (32-key halves)
    static constexpr int VPRE = HD > 128 ? 8 : HD / 16; // V^T operands read ahead of the softmax
    static constexpr int DCH = D / 8;                 // 16-byte chunks per key row
    static constexpr int CPT = BN * DCH / NT;         // chunks per thread per K (and per V) tile
    static constexpr int KSTEPS = D / 32;
    static constexpr int DBLK = D / 16;
};


// BIAS: softcap, ALiBi, a non-positive scale or FP8 descales (scores are
// formed explicitly); PAGED: K/V rows come through the block table; ROT: q is
// rotated (kvcache rotary) as it is loaded. DT_FP8: q, K and V are e4m3fn
// bytes, carried raw through the load registers and widened to bf16 on their
// way into registers (q) and LDS (K/V tiles); the LDS tiles, the MFMAs and
// the output are bf16.
template <int DT, int HD, bool BIAS, bool PAGED, bool ROT>
__global__ void __launch_bounds__(PfCfg<HD>::NT, 1) fa_prefill_kernel(FwdArgs a) {
    using C = PfCfg<HD>;
    constexpr int D = C::D, RB = C::RB, NW = C::NW, NT = C::NT, BM = C::BM, BN = C::BN, DCH = C::DCH,
                  CPT = C::CPT, KSTEPS = C::KSTEPS, DBLK = C::DBLK, VPRE = C::VPRE;
    constexpr bool F8 = DT == DT_FP8;
    using ET = std::conditional_t<F8, uint8_t, uint16_t>;  // stored element
    using RT = std::conditional_t<F8, u32x2, u32x4>;       // 8 stored elements
    static_assert(!F8 || (BIAS && !ROT), "FP8 runs the explicit-score path, without rotary");
    using pf::kLazy;
    __shared__ __attribute__((aligned(16))) uint16_t s_k[2][BN * D];
    __shared__ __attribute__((aligned(16))) uint16_t s_v[2][BN * D];
    __shared__ int s_pref[kMaxBatchLds + 1];
    __shared__ long long s_red[2 * NW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, G = lane >> 4;

    int total, chunk_auto;
    build_schedule<BM, BN, NT, NW>(a, s_pref, s_red, total, chunk_auto);

    // LDS swizzles for the row length (128-byte rows at head dim 64)
    auto swzk = [](int r, int c) { return HD == 64 ? swz_k64(r, c) : swz_k(r, c); };
    auto swzv = [](int r, int c) { return HD == 64 ? swz_v64(r, c) : swz_v(r, c); };
    // loop-invariant LDS offsets (elements)
    int offk[KSTEPS];
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) offk[s] = li * D + (swzk(li, G * KSTEPS + s) << 3);
    const int r4 = li >> 2, c4 = li & 3;
    int offv[DBLK];
#pragma unroll
    for (int db = 0; db < DBLK; ++db)
        offv[db] = (4 * G + r4) * D + (swzv(4 * G + r4, 2 * db + (c4 >> 1)) << 3) + (c4 & 1) * 4;
    const int dch = tid & (DCH - 1), kk0 = tid / DCH;
    const int offsk = kk0 * D + (swzk(kk0, dch) << 3);   // + u*(NT/DCH)*D for chunk u
    const int offsv = kk0 * D + (swzv(kk0, dch) << 3);

    const ET* qp = static_cast<const ET*>(a.q);
    const ET* kp = static_cast<const ET*>(a.k);
    const ET* vp = static_cast<const ET*>(a.v);
    uint16_t* op = static_cast<uint16_t*>(a.out);
    const float cs = a.scale_log2;

    // Pass k takes item k * grid + blockIdx.x, in the other direction on odd
    // passes, so a workgroup's heavy item of one pass pairs with a light one of
    // the next (items are numbered heaviest first within a sequence).
    for (int k = 0; k * (int)gridDim.x < total; ++k) {
        const int w = k * (int)gridDim.x + ((k & 1) ? (int)gridDim.x - 1 - (int)blockIdx.x : (int)blockIdx.x);
        if (w >= total) continue;
        // ---- decode the work item ------------------------------------------------------
        int bl = 0, bh = a.B;
        while (bh - bl > 1) {
            int mid = (bl + bh) >> 1;
            if (s_pref[mid] <= w) bl = mid; else bh = mid;
        }
        const int b = bl;
        BatchInfo bi;
        batch_info<BM>(a, b, bi);
        int ns, chunk;
        split_of(a, bi.hi - bi.lo, chunk_auto, ns, chunk);
        // kv head fastest: the Hk items of one row tile run side by side and
        // stream the same cache rows (heads are interleaved per token in HBM)
        const int local = w - s_pref[b];
        const int hk = local % a.Hk;
        const int split = (local / a.Hk) % ns;
        const int mt_r = local / a.Hk / ns;
        const int mt = bi.mt - 1 - mt_r;  // heaviest causal tiles first
        const bool final_out = ns == 1;
        const int crow = a.batch_idx ? min(max(a.batch_idx[b], 0), (a.block_table ? a.bt_rows : a.batch_cache) - 1) : b;
        const int g = a.g;
        const int diag0 = bi.sk - bi.sq;  // key on the diagonal of query 0 (bottom-right aligned)

        const int tile_row0 = mt * BM;
        const int tile_rows = min(BM, bi.rows - tile_row0);
        int k_lo, k_hi;
        {
            const int i_lo = tile_row0 / g, i_hi = (tile_row0 + tile_rows - 1) / g;
            k_lo = max(0, key_lo(i_lo + diag0, a.wl, a.chunk));
            k_hi = min(bi.sk, key_hi(i_hi + diag0, a.wr, a.chunk) + 1);
            if (ns > 1) {
                const int c0 = bi.lo + split * chunk;
                k_lo = max(k_lo, c0);
                k_hi = min(k_hi, c0 + chunk);
            }
            if (k_hi < k_lo) k_hi = k_lo;
        }
        const int ntiles = (k_hi - k_lo + BN - 1) / BN;

        const int wrow0 = tile_row0 + wave * RB * 16;
        const int wrows = min(RB * 16, bi.rows - wrow0);
        const bool wave_live = wrows > 0;
        const int wi_lo = wave_live ? wrow0 / g : 0;
        const int wi_hi = wave_live ? (wrow0 + wrows - 1) / g : 0;
        // keys visible to some row of the wave: [w_lo, w_hi]; to every row: [f_lo, f_hi]
        const int w_lo = key_lo(wi_lo + diag0, a.wl, a.chunk), w_hi = key_hi(wi_hi + diag0, a.wr, a.chunk);
        const int f_lo = key_lo(wi_hi + diag0, a.wl, a.chunk), f_hi = key_hi(wi_lo + diag0, a.wr, a.chunk);

        // ---- K/V tiles: registers -> double-buffered LDS ----------------------------------
        RT kr[CPT], vr[CPT];
        // per-item row bases: token j of this kv head lives at base + j * si
        // (contiguous / varlen) or at base + blk * sb + (j % page) * si (paged)
        const int kvh = hk / a.kvdiv;  // kv head of this row tile's query heads
        const ET* kb0 = kp + (int64_t)kvh * a.k_sh + dch * 8;
        const ET* vb0 = vp + (int64_t)kvh * a.v_sh + dch * 8;
        // FP8: scores scale by q_descale * k_descale, the output by v_descale
        float sc_qk = a.scale, sc_v = 1.f;
        if constexpr (F8) {
            sc_qk = a.scale * descale_at(a.qd, a.qd_sb, a.qd_sh, b, kvh) * descale_at(a.kd, a.kd_sb, a.kd_sh, b, kvh);
            sc_v = descale_at(a.vd, a.vd_sb, a.vd_sh, b, kvh);
        }
        const int* btrow = nullptr;
        if constexpr (PAGED) {
            btrow = a.block_table + (int64_t)crow * a.bt_stride;
        } else {
            const int64_t row0k = a.cu_seqlens_k ? (int64_t)a.cu_seqlens_k[b] * a.k_si
                                                 : (int64_t)crow * a.k_sb + (int64_t)bi.lp * a.k_si;
            const int64_t row0v = a.cu_seqlens_k ? (int64_t)a.cu_seqlens_k[b] * a.v_si
                                                 : (int64_t)crow * a.v_sb + (int64_t)bi.lp * a.v_si;
            kb0 += row0k;
            vb0 += row0v;
        }
        // contiguous / varlen: this thread's key rows of the next tile as
        // element offsets from kb0 / vb0, moved BN keys on per load_tile call
        // (the calls load the tiles at k_lo, k_lo + BN, ... in that order), so
        // the tile loop does no 64-bit products
        [[maybe_unused]] int64_t kcur[CPT], vcur[CPT], kstep = 0, vstep = 0;
        if constexpr (!PAGED) {
#pragma unroll
            for (int u = 0; u < CPT; ++u) {
                const int j = k_lo + kk0 + u * (NT / DCH);
                kcur[u] = (int64_t)j * a.k_si;
                vcur[u] = (int64_t)j * a.v_si;
            }
            kstep = (int64_t)BN * a.k_si;
            vstep = (int64_t)BN * a.v_si;
        }
        auto load_tile = [&](int t0) {
#pragma unroll
            for (int u = 0; u < CPT; ++u) {
                const int j = t0 + kk0 + u * (NT / DCH);
                if (j < k_hi && dch * 8 < a.hd) {
                    const ET* kpr;
                    const ET* vpr;
                    if constexpr (PAGED) {
                        const int pg = a.page_shift >= 0 ? j >> a.page_shift : j / a.page;
                        const int inp = a.page_shift >= 0 ? j & (a.page - 1) : j % a.page;
                        const int blk = min(max(btrow[pg], 0), a.num_blocks - 1);
                        kpr = kb0 + (int64_t)blk * a.k_sb + (int64_t)inp * a.k_si;
                        vpr = vb0 + (int64_t)blk * a.v_sb + (int64_t)inp * a.v_si;
                    } else {
                        kpr = kb0 + kcur[u];
                        vpr = vb0 + vcur[u];
                    }
                    kr[u] = *reinterpret_cast<const RT*>(kpr);
                    vr[u] = *reinterpret_cast<const RT*>(vpr);
                } else {
                    kr[u] = RT{};
                    vr[u] = RT{};
                }
                if constexpr (!PAGED) {
                    kcur[u] += kstep;
                    vcur[u] += vstep;
                }
            }
        };
        auto widen = [](RT x) -> u32x4 {
            if constexpr (F8) return fp8x8_to_bf16(x);
            else return x;
        };
        auto store_tile = [&](int buf) {
#pragma unroll
            for (int u = 0; u < CPT; ++u) {
                *reinterpret_cast<u32x4*>(&s_k[buf][offsk + u * (NT / DCH) * D]) = widen(kr[u]);
                *reinterpret_cast<u32x4*>(&s_v[buf][offsv + u * (NT / DCH) * D]) = widen(vr[u]);
            }
        };

        // ---- Q operands (B of S^T = K.Q^T), dims permuted by lane group --------------------
        u32x4 qreg[RB][KSTEPS];
        float slope[RB];
        int qi[RB];
        [[maybe_unused]] const ET* qrows[RB];
        [[maybe_unused]] bool qok[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int r = wrow0 + rb * 16 + li;
            const bool ok = r < bi.rows;
            const int i = ok ? r / g : 0;
            const int h = hk * g + (ok ? r % g : 0);
            qi[rb] = i;
            slope[rb] = (BIAS && a.alibi && ok) ? a.alibi[(int64_t)b * a.alibi_sb + h] : 0.f;
            const ET* qrow = a.cu_seqlens_q
                                 ? qp + ((int64_t)a.cu_seqlens_q[b] + i) * a.q_si + (int64_t)h * a.q_sh
                                 : qp + (int64_t)b * a.q_sb + (int64_t)i * a.q_si + (int64_t)h * a.q_sh;
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s)
                qreg[rb][s] = ok && (G * KSTEPS + s) * 8 < a.hd ? widen(*reinterpret_cast<const RT*>(qrow + (G * KSTEPS + s) * 8))
                                                                : u32x4{0u, 0u, 0u, 0u};
            qrows[rb] = qrow;
            qok[rb] = ok;
        }
        // each row's visible keys [rlo, rhi] (before the clamp to k_hi)
        int rlo[RB], rhi[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            rlo[rb] = key_lo(qi[rb] + diag0, a.wl, a.chunk);
            rhi[rb] = key_hi(qi[rb] + diag0, a.wr, a.chunk);
        }
        if constexpr (ROT) {
            // q[b, i] is rotated at cache_seqlens[b] (+ i when causal or local).
            // The rotary arguments are read from the argument block here (the
            // empty asm hides that they are loop invariant), so they hold no
            // scalar registers across the tile loop, where every scalar
            // register is taken. FwdArgs is the kernel's only argument.
            auto kseg = __builtin_amdgcn_kernarg_segment_ptr();
            asm volatile("" : "+s"(kseg));
            const FwdArgs* rk = (const FwdArgs*)kseg;
            const int rot_rd = rk->rot_dim;
            const bool rot_inter = rk->rot_interleaved != 0;
            const int clast = (rot_rd >> 3) - 1;
            // Every operand load is issued before any rotation (chunks past
            // rotary_dim load the last rotated chunk's operands and keep q),
            // so the q rows cost one memory round trip, and that trip overlaps
            // the first K/V tile's.
            auto rotate_q = [&](auto inter_tag) {
                constexpr bool INTER = decltype(inter_tag)::value;
                RopeOps rop[RB][KSTEPS];
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    int pos = (rk->rot_pos ? rk->rot_pos[b] : bi.len0) + (rk->rot_same_pos ? 0 : qi[rb]);
                    pos = min(max(pos, 0), rk->seqlen_ro - 1);
                    const uint16_t* crow_c = static_cast<const uint16_t*>(rk->rot_cos) + (int64_t)pos * (rot_rd >> 1);
                    const uint16_t* crow_s = static_cast<const uint16_t*>(rk->rot_sin) + (int64_t)pos * (rot_rd >> 1);
#pragma unroll
                    for (int s = 0; s < KSTEPS; ++s)
                        rop[rb][s] = rope_load(qrows[rb], min(G * KSTEPS + s, clast), rot_rd, INTER, crow_c, crow_s);
                }
                // the first K/V tile's loads go out before the rotation, which
                // then runs under their latency
                if (ntiles > 0) load_tile(k_lo);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int s = 0; s < KSTEPS; ++s) {
                        const int c = G * KSTEPS + s;
                        const u32x4 rq = rope_apply<DT>(qreg[rb][s], rop[rb][s], c, rot_rd, INTER);
                        if (qok[rb] && c <= clast) qreg[rb][s] = rq;
                    }
            };
            if (rot_inter) rotate_q(std::true_type{});
            else rotate_q(std::false_type{});
        }

        // Retire the q loads here. Otherwise the wait-count tracking merges
        // them with the K/V prefetch at the tile loop's back edge and waits
        // for that prefetch (vmcnt(0)) before every QK product.
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt, lgkmcnt unconstrained

        f32x4 oacc[RB][DBLK];
        float m_run[RB], l_run[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            m_run[rb] = -1e30f;  // finite floor: exp2(x - m) never forms inf - inf
            l_run[rb] = 0.f;
#pragma unroll
            for (int db = 0; db < DBLK; ++db) oacc[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
        }

        // 32 keys (half of the LDS tile at key offset 32*hh) for this wave's 64
        // rows; MASK: apply the per-key test
        auto tile = [&](int buf, int hh, int s0, auto mask_tag) {
            constexpr bool MASK = decltype(mask_tag)::value;
            f32x4 sacc[RB][2];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                sacc[rb][0] = f32x4{0.f, 0.f, 0.f, 0.f};
                sacc[rb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    const u32x4 av = *reinterpret_cast<const u32x4*>(&s_k[buf][offk[s] + (hh * 32 + kb * 16) * D]);
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) sacc[rb][kb] = mfma16x16x32<DT>(av, qreg[rb][s], sacc[rb][kb]);
                }
            }
            // V^T operands for this half tile (transpose reads), issued now so
            // the LDS latency hides under the softmax below; past VPRE blocks
            // (head dim 256) each read is issued one window ahead of its use
            auto read_vt = [&](int db) {
                const s16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)&s_v[buf][offv[db] + (32 * hh) * D]);
                const s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)&s_v[buf][offv[db] + (32 * hh + 16) * D]);
                const u32x2 l2 = __builtin_bit_cast(u32x2, lo4);
                const u32x2 h2 = __builtin_bit_cast(u32x2, hi4);
                return u32x4{l2[0], l2[1], h2[0], h2[1]};
            };
            u32x4 vt[VPRE];
#pragma unroll
            for (int db = 0; db < VPRE; ++db) vt[db] = read_vt(db);
            // scores (log2 units when BIAS; raw otherwise, scaled inside exp2's FMA)
            float xmax[RB];
            bool need = false;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                float mx = -INFINITY;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float x = sacc[rb][kb][e];
                        const int j = s0 + kb * 16 + G * 4 + e;
                        if constexpr (BIAS) {
                            float y = x * sc_qk;
                            if (a.softcap > 0.f) y = a.softcap * fast_tanh(y * (1.f / a.softcap));
                            if (a.alibi) {
                                int dist = qi[rb] + diag0 - j;
                                dist = dist < 0 ? -dist : dist;
                                y -= slope[rb] * (float)dist;
                            }
                            x = y * kLog2e;
                        }
                        if constexpr (MASK) {
                            const bool vis = j < k_hi && j >= rlo[rb] && j <= rhi[rb];
                            x = vis ? x : -INFINITY;
                        }
                        sacc[rb][kb][e] = x;
                        mx = fmaxf(mx, x);
                    }
                xmax[rb] = BIAS ? mx : mx * cs;
                need |= xmax[rb] > m_run[rb] + kLazy;
            }
            if (__ballot(need)) {
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    const float mn = fmaxf(m_run[rb], wave_max16x4(xmax[rb]));
                    const float alpha = fast_exp2(m_run[rb] - mn);
                    m_run[rb] = mn;
                    l_run[rb] *= alpha;
#pragma unroll
                    for (int db = 0; db < DBLK; ++db) {
                        f32x4 o = oacc[rb][db];
                        asm volatile("" : "+v"(o));  // pins the multiply inside this branch
                        oacc[rb][db] = o * alpha;
                    }
                }
            }
            u32x4 pk[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                float p[2][4], ps = 0.f;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float x = sacc[rb][kb][e];
                        p[kb][e] = fast_exp2(BIAS ? x - m_run[rb] : __builtin_fmaf(x, cs, -m_run[rb]));
                        ps += p[kb][e];
                    }
                l_run[rb] += ps;
                f32x8 v8 = {p[0][0], p[0][1], p[0][2], p[0][3], p[1][0], p[1][1], p[1][2], p[1][3]};
                pk[rb] = pack8<DT>(v8);
            }
            // O^T += V^T . P^T, issued at raised wave priority: while this wave
            // streams its PV products, the SIMD's other wave (in its QK
            // products or softmax) only fills the issue slots between them.
            // Measured on the c4 shape: 1010 -> 935..965 us; raising it for
            // the QK products as well is slower (1030 us).
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int db = 0; db < DBLK; ++db) {
                const u32x4 cur = vt[db % VPRE];
                if (db + VPRE < DBLK) vt[db % VPRE] = read_vt(db + VPRE);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) oacc[rb][db] = mfma16x16x32<DT>(cur, pk[rb], oacc[rb][db]);
            }
            __builtin_amdgcn_s_setprio(0);
        };

        if (ntiles > 0) {
            if constexpr (!ROT) load_tile(k_lo);  // ROT issued it with the q rotation
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
                    if (h0 > w_hi || h1 - 1 < w_lo || h0 >= k_hi) continue;
                    const bool full = h1 <= k_hi && h0 >= f_lo && h1 - 1 <= f_hi;
                    if (full) tile(buf, hh, h0, std::integral_constant<bool, false>{});
                    else tile(buf, hh, h0, std::integral_constant<bool, true>{});
                }
            }
            if (t + 1 < ntiles) store_tile(buf ^ 1);
            if (t + 2 < ntiles) load_tile(k_lo + (t + 2) * BN);
            __syncthreads();
        }

        // ---- epilogue -----------------------------------------------------------------------
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int r = wrow0 + rb * 16 + li;
            const float lrow = wave_sum16x4(l_run[rb]);
            const bool nonempty = lrow > 0.f;
            const float inv = nonempty ? (F8 ? sc_v / lrow : 1.f / lrow) : 0.f;
            const float lse = nonempty ? (m_run[rb] + fast_log2(lrow)) * kLn2 : (final_out ? INFINITY : -INFINITY);
            if (r < bi.rows) {
                const int i = r / g, h = hk * g + r % g;
                if (final_out) {
                    uint16_t* orow = a.cu_seqlens_q
                                         ? op + ((int64_t)a.cu_seqlens_q[b] + i) * a.o_si + (int64_t)h * a.o_sh
                                         : op + (int64_t)b * a.o_sb + (int64_t)i * a.o_si + (int64_t)h * a.o_sh;
#pragma unroll
                    for (int db = 0; db < DBLK; ++db) {
                        if (16 * db + 4 * G >= a.hd) continue;
                        const f32x4 o = oacc[rb][db] * inv;
                        uint16_t h4[4] = {f32_to_16<DT>(o[0]), f32_to_16<DT>(o[1]), f32_to_16<DT>(o[2]), f32_to_16<DT>(o[3])};
                        *reinterpret_cast<u32x2*>(orow + 16 * db + 4 * G) = __builtin_bit_cast(u32x2, h4);
                    }
                    if (G == 0) {
                        const int64_t off = a.cu_seqlens_q ? (int64_t)h * a.lse_sh + a.cu_seqlens_q[b] + i
                                                           : (int64_t)b * a.lse_sb + (int64_t)h * a.lse_sh + i;
                        a.lse[off] = lse;
                    }
                } else {
                    const int64_t prow = (int64_t)w * BM + (r - tile_row0);
#pragma unroll
                    for (int db = 0; db < DBLK; ++db)
                        *reinterpret_cast<f32x4*>(a.part_o + prow * D + 16 * db + 4 * G) = oacc[rb][db] * inv;
                    if (G == 0) a.part_lse[prow] = lse;
                }
            }
        }
    }
}

// Split-KV merge as its own launch: one thread per (row, 8 dims) of a split
// row tile; the per-batch plan comes from the attention kernel's sched table.
template <int DT, int D, int BM>
__global__ void __launch_bounds__(256) fa_merge_kernel(FwdArgs a) {
    constexpr int DCH = D / 8;
    constexpr int RPB = 256 / DCH;                // rows per block
    constexpr int BPT = (BM + RPB - 1) / RPB;     // blocks per tile
    const int blk = blockIdx.x % BPT;
    const int tile = blockIdx.x / BPT;
    const int hk = tile % a.Hk;
    const int bm = tile / a.Hk;
    const int mt = bm % a.mt_max, b = bm / a.mt_max;
    if (b >= a.B) return;
    const int ns = a.sched[a.B + 1 + b];
    if (ns <= 1) return;
    int sq = a.cu_seqlens_q ? a.cu_seqlens_q[b + 1] - a.cu_seqlens_q[b] : a.Sq;
    sq = min(max(sq, 0), a.Sq);
    const int rows = sq * a.g;
    const int mt_b = (rows + BM - 1) / BM;
    if (mt >= mt_b) return;
    const int mt_r = mt_b - 1 - mt;
    const int rr = blk * RPB + threadIdx.x / DCH;
    const int d0 = (threadIdx.x % DCH) * 8;
    const int row0 = mt * BM;
    if (rr >= min(BM, rows - row0)) return;
    const int sst = a.Hk;  // split s of this tile is item w0 + s * Hk
    const int w0 = a.sched[b] + mt_r * ns * a.Hk + hk;
    float m = -INFINITY;
    for (int s = 0; s < ns; ++s) m = fmaxf(m, a.part_lse[(int64_t)(w0 + s * sst) * BM + rr]);
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    float lse = INFINITY;
    if (m != -INFINITY) {
        float sum = 0.f;
        for (int s = 0; s < ns; ++s) {
            const int64_t prow = (int64_t)(w0 + s * sst) * BM + rr;
            const float wgt = fast_exp2((a.part_lse[prow] - m) * kLog2e);
            sum += wgt;
            acc0 += *reinterpret_cast<const f32x4*>(a.part_o + prow * D + d0) * wgt;
            acc1 += *reinterpret_cast<const f32x4*>(a.part_o + prow * D + d0 + 4) * wgt;
        }
        const float inv = 1.f / sum;
        acc0 *= inv;
        acc1 *= inv;
        lse = m + fast_log2(sum) * kLn2;
    }
    const int r = row0 + rr;
    const int i = r / a.g, h = hk * a.g + r % a.g;
    uint16_t* op = static_cast<uint16_t*>(a.out);
    uint16_t* orow;
    if (a.cu_seqlens_q) orow = op + ((int64_t)a.cu_seqlens_q[b] + i) * a.o_si + (int64_t)h * a.o_sh;
    else orow = op + (int64_t)b * a.o_sb + (int64_t)i * a.o_si + (int64_t)h * a.o_sh;
    uint16_t h8[8] = {f32_to_16<DT>(acc0[0]), f32_to_16<DT>(acc0[1]), f32_to_16<DT>(acc0[2]), f32_to_16<DT>(acc0[3]),
                      f32_to_16<DT>(acc1[0]), f32_to_16<DT>(acc1[1]), f32_to_16<DT>(acc1[2]), f32_to_16<DT>(acc1[3])};
    if (d0 < a.hd) *reinterpret_cast<u32x4*>(orow + d0) = __builtin_bit_cast(u32x4, h8);
    if (d0 == 0) {
        int64_t lo_off = a.cu_seqlens_q ? (int64_t)h * a.lse_sh + a.cu_seqlens_q[b] + i
                                        : (int64_t)b * a.lse_sb + (int64_t)h * a.lse_sh + i;
        a.lse[lo_off] = lse;
    }
}

// Standalone merge of caller-provided partials (the v3 flash_attn_combine):
// out_partial (S, R, Dv), lse_partial (S, R); one thread per (row, 4 dims).
template <int OUT>
__global__ void __launch_bounds__(256) fa_combine_flat_kernel(const float* __restrict__ po, const float* __restrict__ pl,
                                                              int S, int64_t R, int Dv, void* out, int64_t ors,
                                                              float* lse) {
    const int q4 = Dv / 4;
    const int64_t n = R * q4;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = idx / q4;
        const int d0 = (int)(idx % q4) * 4;
        float m = -INFINITY;
        for (int s = 0; s < S; ++s) {
            float v = pl[(int64_t)s * R + r];
            if (v > m && v != INFINITY) m = v;
        }
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        float l = INFINITY;
        if (m != -INFINITY) {
            float sum = 0.f;
            for (int s = 0; s < S; ++s) {
                float v = pl[(int64_t)s * R + r];
                if (v != -INFINITY && v != INFINITY) sum += fast_exp2((v - m) * kLog2e);
            }
            l = m + fast_log2(sum) * kLn2;
            for (int s = 0; s < S; ++s) {
                float v = pl[(int64_t)s * R + r];
                if (v == -INFINITY || v == INFINITY) continue;
                acc += *reinterpret_cast<const f32x4*>(po + ((int64_t)s * R + r) * Dv + d0) * fast_exp2((v - l) * kLog2e);
            }
        }
        if constexpr (OUT == 2) {
            *reinterpret_cast<f32x4*>(static_cast<float*>(out) + r * ors + d0) = acc;
        } else {
            uint16_t h4[4] = {f32_to_16<OUT>(acc[0]), f32_to_16<OUT>(acc[1]), f32_to_16<OUT>(acc[2]),
                              f32_to_16<OUT>(acc[3])};
            *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(out) + r * ors + d0) = __builtin_bit_cast(u32x2, h4);
        }
        if (d0 == 0 && lse) lse[r] = l;
    }
}

// ---- host-side launchers (called from fa_api.cpp) -------------------------------------
int fwd_tile_rows(int d) { return d > 128 ? PfCfg<256>::BM : d > 64 ? PfCfg<128>::BM : PfCfg<64>::BM; }
int fwd_tile_keys(int d) { return d > 128 ? PfCfg<256>::BN : d > 64 ? PfCfg<128>::BN : PfCfg<64>::BN; }

template <int DT, int HD, bool BIAS, bool ROT>
static void launch_prefill_r(const FwdArgs& a, int grid, hipStream_t stream) {
    constexpr int NT = PfCfg<HD>::NT;
    if (a.block_table) hipLaunchKernelGGL((fa_prefill_kernel<DT, HD, BIAS, true, ROT>), dim3(grid), dim3(NT), 0, stream, a);
    else hipLaunchKernelGGL((fa_prefill_kernel<DT, HD, BIAS, false, ROT>), dim3(grid), dim3(NT), 0, stream, a);
}

template <int DT, int HD, bool BIAS>
static void launch_prefill_b(const FwdArgs& a, int grid, hipStream_t stream) {
    if (a.rot_cos) launch_prefill_r<DT, HD, BIAS, true>(a, grid, stream);
    else launch_prefill_r<DT, HD, BIAS, false>(a, grid, stream);
}

template <int HD>
static void launch_prefill_d(const FwdArgs& a, int dtype, int grid, hipStream_t stream) {
    const bool bias = a.softcap > 0.f || a.alibi != nullptr || !(a.scale > 0.f);
    if (dtype == DT_BF16) {
        if (bias) launch_prefill_b<DT_BF16, HD, true>(a, grid, stream);
        else launch_prefill_b<DT_BF16, HD, false>(a, grid, stream);
    } else if (dtype == DT_FP8) {
        // descales of any sign: the explicit-score path; no rotary with FP8
        launch_prefill_r<DT_FP8, HD, true, false>(a, grid, stream);
    } else {
        if (bias) launch_prefill_b<DT_FP16, HD, true>(a, grid, stream);
        else launch_prefill_b<DT_FP16, HD, false>(a, grid, stream);
    }
}

// d: the kernel head dim, 64, 128 or 256 (a.hd <= d is the head dim in memory)
hipError_t launch_fwd(const FwdArgs& a, int dtype, int d, int grid, hipStream_t stream) {
    if (d == 64) launch_prefill_d<64>(a, dtype, grid, stream);
    else if (d == 128) launch_prefill_d<128>(a, dtype, grid, stream);
    else if (d == 256) launch_prefill_d<256>(a, dtype, grid, stream);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

template <int HD>
static void launch_merge_d(const FwdArgs& a, int dtype, hipStream_t stream) {
    constexpr int BM = PfCfg<HD>::BM;
    constexpr int RPB = 256 / (HD / 8);
    const int64_t grid = (int64_t)a.B * a.mt_max * a.Hk * ((BM + RPB - 1) / RPB);
    if (dtype == DT_BF16 || dtype == DT_FP8)  // FP8 inputs give a bf16 output
        hipLaunchKernelGGL((fa_merge_kernel<DT_BF16, HD, BM>), dim3(grid), dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((fa_merge_kernel<DT_FP16, HD, BM>), dim3(grid), dim3(256), 0, stream, a);
}

hipError_t launch_merge(const FwdArgs& a, int dtype, int d, hipStream_t stream) {
    if (d == 64) launch_merge_d<64>(a, dtype, stream);
    else if (d == 128) launch_merge_d<128>(a, dtype, stream);
    else if (d == 256) launch_merge_d<256>(a, dtype, stream);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_combine_flat(const float* po, const float* pl, int S, int64_t R, int Dv, void* out, int64_t ors,
                               int out_dtype, float* lse, hipStream_t stream) {
    int64_t n = R * (Dv / 4);
    int grid = (int)((n + 255) / 256);
    if (grid > 16384) grid = 16384;
    if (grid < 1) grid = 1;
    if (out_dtype == 2)
        hipLaunchKernelGGL(fa_combine_flat_kernel<2>, dim3(grid), dim3(256), 0, stream, po, pl, S, R, Dv, out, ors, lse);
    else if (out_dtype == DT_BF16)
        hipLaunchKernelGGL(fa_combine_flat_kernel<DT_BF16>, dim3(grid), dim3(256), 0, stream, po, pl, S, R, Dv, out, ors, lse);
    else
        hipLaunchKernelGGL(fa_combine_flat_kernel<DT_FP16>, dim3(grid), dim3(256), 0, stream, po, pl, S, R, Dv, out, ors, lse);
    return hipGetLastError();
}

}  // namespace fa
