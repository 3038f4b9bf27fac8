// fa_fwd.hip -- FlashAttention forward for gfx950 (MI355X): attention core,
// in-kernel split-KV scheduler and the log-sum-exp combine.
//
// Reference behaviour being reproduced (paths relative to the reference repo):
//   SplitFuse::FAInfer / runMainLoop  csrc/arch22/flash_attn_npu_v2/mha_fwd_kvcache.cpp:436-966
//   online softmax                    csrc/arch22/flash_attn_npu_v2/online_softmax.hpp:477-803
//   rescale / finalize / LSE          csrc/arch22/flash_attn_npu_v2/rescale_o.hpp:299-534
//   split-KV combine                  csrc/arch22/flash_attn_npu_v2/CombineScale.hpp:76-357
//   split planner                     csrc/arch22/flash_attn_npu_v3/fa_split.h:483-510
// The design is MI355X-native rather than a translation:
//   * Rows of one work tile are (query position, q head) pairs of ONE kv head
//     (GQA packing, row r -> position r / g, head hk*g + r % g), so every K/V
//     byte fetched from HBM serves all g query heads.
//   * S^T = K.Q^T with 16x16x32 MFMA: the accumulator then holds, per lane, one
//     query row and 8 keys, which is exactly the packed P^T operand of
//     O^T = V^T.P^T. The head dimension of Q/K is permuted (lane group G takes
//     dims G*D/4 .. +D/4) so every lane reads 16-byte contiguous chunks.
//   * K and V tiles are staged in LDS with a 16-byte XOR swizzle; V^T operands
//     come from ds_read_b64_tr_b16 (transpose on read).
//   * Online softmax in fp32 in the log2 domain (v_exp_f32); P is rounded to
//     the input dtype before P.V and the row sum uses the fp32 P, as in the
//     reference golden (tests/test_flash_attn_npu_v3.py:29-47,130).
//   * Masks are evaluated arithmetically per tile; fully visible tiles skip the
//     per-element test and fully hidden tiles are skipped.
//   * The split-KV plan is computed by every workgroup from cache_seqlens in
//     LDS (no host round trip); the kernel is persistent over the work list.
#include "fa_common.h"
#include "fa_kernel_args.h"

namespace fa {

constexpr int kMaxBatchLds = 2048;

template <int DT_, int D_, int WR_, int WK_, int RB_, int KW_, int MINB_>
struct Cfg {
    static constexpr int DT = DT_, D = D_, WR = WR_, WK = WK_, RB = RB_, KW = KW_, MINB = MINB_;
    static constexpr int NW = WR * WK;          // waves per workgroup
    static constexpr int NT = NW * 64;          // threads per workgroup
    static constexpr int BM = WR * RB * 16;     // packed rows per work tile
    static constexpr int BN = WK * KW;          // keys per LDS tile
    static constexpr int DCH = D / 8;           // 16-byte chunks per key row
    static constexpr int SWZ = DCH >= 16 ? 15 : DCH - 1;
    static constexpr int CPT = BN * DCH / NT;   // chunks per thread per K (and per V) tile
    static constexpr int KSTEPS = D / 32;
    static constexpr int DBLK = D / 16;
    static_assert((BN * DCH) % NT == 0, "tile chunks must divide over the threads");
    static_assert(KW % 32 == 0, "a wave handles whole 32-key MFMA steps");
    static_assert(D % 32 == 0, "head dim must be a multiple of 32");
};

struct BatchInfo {
    int sq, sk, rows, mt, lo, hi;
};

template <int BM>
__device__ __forceinline__ void batch_info(const FwdArgs& a, int b, BatchInfo& bi) {
    int sq = a.cu_seqlens_q ? a.cu_seqlens_q[b + 1] - a.cu_seqlens_q[b] : a.Sq;
    int sk;
    if (a.seqlens_k) sk = a.seqlens_k[b] + a.seqlen_new;  // cache_seqlens / seqused_k
    else if (a.cu_seqlens_k) sk = a.cu_seqlens_k[b + 1] - a.cu_seqlens_k[b];
    else sk = a.Sk;
    sq = min(max(sq, 0), a.Sq);  // Sq is max_seqlen_q for varlen: bounds the tiles
    sk = min(max(sk, 0), a.kv_capacity);
    bi.sq = sq;
    bi.sk = sk;
    bi.rows = sq * a.g;
    bi.mt = (bi.rows + BM - 1) / BM;
    // union of the keys visible to any row of this sequence
    int lo = a.wl >= 0 ? max(0, sk - sq - a.wl) : 0;
    int hi = a.wr >= 0 ? min(sk, sk - 1 + a.wr + 1) : sk;
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
template <class C>
__device__ void build_schedule(const FwdArgs& a, int* s_pref, long long* s_red, int& total, int& chunk_auto) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    long long work = 0, base = 0;
    for (int b = tid; b < a.B; b += C::NT) {
        BatchInfo bi;
        batch_info<C::BM>(a, b, bi);
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
    for (int w = 0; w < C::NW; ++w) {
        work += s_red[w * 2];
        base += s_red[w * 2 + 1];
    }
    int ca = 0x3fffffff;
    if (a.allow_split && a.num_splits <= 0 && base < a.target_items) {
        long long c = (work + a.target_items - 1) / a.target_items;
        c = c < a.min_chunk ? a.min_chunk : c;
        c = (c + C::BN - 1) / C::BN * C::BN;
        ca = (int)(c > 0x3fffffff ? 0x3fffffff : c);
    }
    chunk_auto = ca;
    for (int b = tid; b < a.B; b += C::NT) {
        BatchInfo bi;
        batch_info<C::BM>(a, b, bi);
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
        for (int b = tid; b <= a.B; b += C::NT) a.sched[b] = s_pref[b];
    }
}

template <class C>
__device__ __forceinline__ const uint16_t* kv_row_ptr(const FwdArgs& a, const uint16_t* base, int64_t sb,
                                                      int64_t si, int64_t sh, int b, int crow, int j, int hk) {
    if (a.block_table) {
        int blk = a.block_table[(int64_t)crow * a.bt_stride + j / a.page];
        blk = min(max(blk, 0), a.num_blocks - 1);
        return base + (int64_t)blk * sb + (int64_t)(j % a.page) * si + (int64_t)hk * sh;
    }
    if (a.cu_seqlens_k) return base + ((int64_t)a.cu_seqlens_k[b] + j) * si + (int64_t)hk * sh;
    return base + (int64_t)crow * sb + (int64_t)j * si + (int64_t)hk * sh;
}

template <class C>
__global__ void __launch_bounds__(C::NT, C::MINB) fa_fwd_kernel(FwdArgs a) {
    constexpr int DT = C::DT, D = C::D, WR = C::WR, WK = C::WK, RB = C::RB, KW = C::KW;
    constexpr int NT = C::NT, BM = C::BM, BN = C::BN, DCH = C::DCH, SWZ = C::SWZ, CPT = C::CPT;
    constexpr int KSTEPS = C::KSTEPS, DBLK = C::DBLK;
    constexpr int KV_ELEMS = BN * D;
    // WK > 1 merges the waves' states through LDS reusing the K/V area.
    constexpr int MERGE_FLOATS = (WK > 1) ? C::NW * 16 * (D + 4) + C::NW * 32 : 0;
    constexpr int KV_BYTES = 2 * KV_ELEMS * 2;
    constexpr int LDS_BYTES = KV_BYTES > MERGE_FLOATS * 4 ? KV_BYTES : MERGE_FLOATS * 4;

    __shared__ __attribute__((aligned(16))) unsigned char s_raw[LDS_BYTES];
    __shared__ int s_pref[kMaxBatchLds + 1];
    __shared__ long long s_red[2 * C::NW];

    uint16_t* s_k = reinterpret_cast<uint16_t*>(s_raw);
    uint16_t* s_v = s_k + KV_ELEMS;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, G = lane >> 4;
    const int wrow = wave % WR, wkey = wave / WR;

    int total, chunk_auto;
    build_schedule<C>(a, s_pref, s_red, total, chunk_auto);

    const uint16_t* qp = static_cast<const uint16_t*>(a.q);
    const uint16_t* kp = static_cast<const uint16_t*>(a.k);
    const uint16_t* vp = static_cast<const uint16_t*>(a.v);

    for (int w = blockIdx.x; w < total; w += gridDim.x) {
        // ---- decode the work item ------------------------------------------------
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
        // kv head fastest: the Hk items of one key chunk run side by side and
        // stream the same cache rows (heads are interleaved per token in HBM)
        const int local = w - s_pref[b];
        const int hk = local % a.Hk;
        const int split = (local / a.Hk) % ns;
        const int mt_r = local / a.Hk / ns;
        const int mt = bi.mt - 1 - mt_r;  // heaviest causal tiles first
        const bool final_out = ns == 1;
        const int crow = a.batch_idx ? min(max(a.batch_idx[b], 0), (a.block_table ? a.bt_rows : a.batch_cache) - 1) : b;
        const int g = a.g;
        const int sq = bi.sq, sk = bi.sk;
        const int diag0 = sk - sq;  // key on the diagonal of query 0 (bottom-right aligned)

        const int tile_row0 = mt * BM;
        const int tile_rows = min(BM, bi.rows - tile_row0);
        int k_lo, k_hi;
        {
            int i_lo = tile_row0 / g, i_hi = (tile_row0 + tile_rows - 1) / g;
            k_lo = a.wl >= 0 ? max(0, i_lo + diag0 - a.wl) : 0;
            k_hi = a.wr >= 0 ? min(sk, i_hi + diag0 + a.wr + 1) : sk;
            if (ns > 1) {
                int c0 = bi.lo + split * chunk;
                k_lo = max(k_lo, c0);
                k_hi = min(k_hi, c0 + chunk);
            }
            if (k_hi < k_lo) k_hi = k_lo;
        }
        const int ntiles = (k_hi - k_lo + BN - 1) / BN;

        // this wave's rows
        const int wrow0 = tile_row0 + wrow * RB * 16;
        const int wrows = min(RB * 16, bi.rows - wrow0);
        const bool wave_live = wrows > 0;
        const int wi_lo = wave_live ? wrow0 / g : 0;
        const int wi_hi = wave_live ? (wrow0 + wrows - 1) / g : 0;

        // ---- Q operands (B of S^T = K.Q^T), dims permuted by lane group ------------
        u32x4 qreg[RB][KSTEPS];
        float slope[RB];
        int qi[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            int r = wrow0 + rb * 16 + li;
            bool ok = r < bi.rows;
            int i = ok ? r / g : 0;
            int h = hk * g + (ok ? r % g : 0);
            qi[rb] = i;
            slope[rb] = (a.alibi && ok) ? a.alibi[(int64_t)b * a.alibi_sb + h] : 0.f;
            const uint16_t* qrow;
            if (a.cu_seqlens_q) qrow = qp + ((int64_t)a.cu_seqlens_q[b] + i) * a.q_si + (int64_t)h * a.q_sh;
            else qrow = qp + (int64_t)b * a.q_sb + (int64_t)i * a.q_si + (int64_t)h * a.q_sh;
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) {
                u32x4 z = {0u, 0u, 0u, 0u};
                qreg[rb][s] = ok ? *reinterpret_cast<const u32x4*>(qrow + (G * KSTEPS + s) * 8) : z;
            }
        }

        f32x4 oacc[RB][DBLK];
        float m_run[RB], l_run[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            m_run[rb] = -INFINITY;
            l_run[rb] = 0.f;
#pragma unroll
            for (int db = 0; db < DBLK; ++db) oacc[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
        }

        // ---- K/V tile pipeline: registers hold the next tile while LDS holds this one
        u32x4 kr[CPT], vr[CPT];
        const int dch = tid % DCH;
        auto load_tile = [&](int t0) {
#pragma unroll
            for (int u = 0; u < CPT; ++u) {
                int kk = (tid + u * NT) / DCH;
                int j = t0 + kk;
                u32x4 z = {0u, 0u, 0u, 0u};
                if (j < k_hi) {
                    const uint16_t* kpr = kv_row_ptr<C>(a, kp, a.k_sb, a.k_si, a.k_sh, b, crow, j, hk);
                    const uint16_t* vpr = kv_row_ptr<C>(a, vp, a.v_sb, a.v_si, a.v_sh, b, crow, j, hk);
                    kr[u] = *reinterpret_cast<const u32x4*>(kpr + dch * 8);
                    vr[u] = *reinterpret_cast<const u32x4*>(vpr + dch * 8);
                } else {
                    kr[u] = z;
                    vr[u] = z;
                }
            }
        };
        if (ntiles > 0) load_tile(k_lo);

        for (int t = 0; t < ntiles; ++t) {
            const int t0 = k_lo + t * BN;
            __syncthreads();
#pragma unroll
            for (int u = 0; u < CPT; ++u) {
                int kk = (tid + u * NT) / DCH;
                int off = kk * D + ((dch ^ (kk & SWZ)) << 3);
                *reinterpret_cast<u32x4*>(s_k + off) = kr[u];
                *reinterpret_cast<u32x4*>(s_v + off) = vr[u];
            }
            if (t + 1 < ntiles) load_tile(t0 + BN);
            __syncthreads();

            // ---- this wave's key slice -------------------------------------------
            const int ws = wkey * KW;  // offset inside the LDS tile
            const int s0 = t0 + ws, s1 = s0 + KW;
            bool skip = !wave_live || s0 >= k_hi;
            if (a.wr >= 0 && s0 > wi_hi + diag0 + a.wr) skip = true;
            if (a.wl >= 0 && s1 - 1 < wi_lo + diag0 - a.wl) skip = true;
            if (skip) continue;
            bool full = s1 <= k_hi;
            if (a.wl >= 0 && s0 < wi_hi + diag0 - a.wl) full = false;
            if (a.wr >= 0 && s1 - 1 > wi_lo + diag0 + a.wr) full = false;

            f32x4 sacc[RB][KW / 16];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int kb = 0; kb < KW / 16; ++kb) sacc[rb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) {
#pragma unroll
                for (int kb = 0; kb < KW / 16; ++kb) {
                    int kk = ws + kb * 16 + li;
                    int ch = G * KSTEPS + s;
                    u32x4 av = *reinterpret_cast<const u32x4*>(s_k + kk * D + ((ch ^ (kk & SWZ)) << 3));
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) sacc[rb][kb] = mfma16x16x32<DT>(av, qreg[rb][s], sacc[rb][kb]);
                }
            }

            // ---- online softmax (log2 domain) ----------------------------------------
            u32x4 pk[RB][KW / 32];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                float x[KW / 16][4];
                const bool plain = a.softcap <= 0.f && a.alibi == nullptr;
#pragma unroll
                for (int kb = 0; kb < KW / 16; ++kb) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float sv = sacc[rb][kb][e];
                        float xv;
                        if (plain) {
                            xv = sv * a.scale_log2;
                        } else {
                            float y = sv * a.scale;
                            if (a.softcap > 0.f) y = a.softcap * tanhf(y / a.softcap);
                            if (a.alibi) {
                                int j = s0 + kb * 16 + G * 4 + e;
                                int dist = qi[rb] + diag0 - j;
                                dist = dist < 0 ? -dist : dist;
                                y -= slope[rb] * (float)dist;
                            }
                            xv = y * kLog2e;
                        }
                        x[kb][e] = xv;
                    }
                }
                if (!full) {
                    const int dg = qi[rb] + diag0;
#pragma unroll
                    for (int kb = 0; kb < KW / 16; ++kb) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            int j = s0 + kb * 16 + G * 4 + e;
                            bool vis = j < k_hi;
                            if (a.wl >= 0 && j < dg - a.wl) vis = false;
                            if (a.wr >= 0 && j > dg + a.wr) vis = false;
                            x[kb][e] = vis ? x[kb][e] : -INFINITY;
                        }
                    }
                }
                float tmax = -INFINITY;
#pragma unroll
                for (int kb = 0; kb < KW / 16; ++kb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) tmax = fmaxf(tmax, x[kb][e]);
                tmax = wave_max16x4(tmax);
                const float m_new = fmaxf(m_run[rb], tmax);
                const float m_use = m_new == -INFINITY ? 0.f : m_new;
                const float alpha = fast_exp2(m_run[rb] - m_use);
                m_run[rb] = m_new;
                float psum = 0.f;
                float p[KW / 16][4];
#pragma unroll
                for (int kb = 0; kb < KW / 16; ++kb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        p[kb][e] = fast_exp2(x[kb][e] - m_use);
                        psum += p[kb][e];
                    }
                l_run[rb] = l_run[rb] * alpha + psum;
#pragma unroll
                for (int db = 0; db < DBLK; ++db) oacc[rb][db] *= alpha;
#pragma unroll
                for (int j = 0; j < KW / 32; ++j) {
                    f32x8 v8 = {p[2 * j][0], p[2 * j][1], p[2 * j][2], p[2 * j][3],
                                p[2 * j + 1][0], p[2 * j + 1][1], p[2 * j + 1][2], p[2 * j + 1][3]};
                    pk[rb][j] = pack8<DT>(v8);
                }
            }

            // ---- O^T += V^T . P^T  (V^T from transpose reads) --------------------------
            const int r4 = li >> 2, c4 = li & 3;
#pragma unroll
            for (int j = 0; j < KW / 32; ++j) {
                const int ka = ws + 32 * j + 4 * G + r4;
                const int kb2 = ka + 16;
#pragma unroll
                for (int db = 0; db < DBLK; ++db) {
                    const int ch = 2 * db + (c4 >> 1);
                    const int off = (c4 & 1) * 4;
                    s16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_s16x4*)(s_v + ka * D + ((ch ^ (ka & SWZ)) << 3) + off));
                    s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_s16x4*)(s_v + kb2 * D + ((ch ^ (kb2 & SWZ)) << 3) + off));
                    u32x2 l2 = __builtin_bit_cast(u32x2, lo4);
                    u32x2 h2 = __builtin_bit_cast(u32x2, hi4);
                    u32x4 av = {l2[0], l2[1], h2[0], h2[1]};
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) oacc[rb][db] = mfma16x16x32<DT>(av, pk[rb][j], oacc[rb][db]);
                }
            }
        }

        // ---- epilogue --------------------------------------------------------------
        uint16_t* op = static_cast<uint16_t*>(a.out);
        if constexpr (WK == 1) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const int r = wrow0 + rb * 16 + li;
                const float lrow = wave_sum16x4(l_run[rb]);
                const bool nonempty = lrow > 0.f;
                const float inv = nonempty ? 1.f / lrow : 0.f;
                const float lse = nonempty ? (m_run[rb] + fast_log2(lrow)) * kLn2 : (final_out ? INFINITY : -INFINITY);
                if (r < bi.rows) {
                    const int i = r / g, h = hk * g + r % g;
                    if (final_out) {
                        uint16_t* orow;
                        if (a.cu_seqlens_q) orow = op + ((int64_t)a.cu_seqlens_q[b] + i) * a.o_si + (int64_t)h * a.o_sh;
                        else orow = op + (int64_t)b * a.o_sb + (int64_t)i * a.o_si + (int64_t)h * a.o_sh;
#pragma unroll
                        for (int db = 0; db < DBLK; ++db) {
                            f32x4 o = oacc[rb][db] * inv;
                            uint16_t h4[4] = {f32_to_16<DT>(o[0]), f32_to_16<DT>(o[1]), f32_to_16<DT>(o[2]),
                                              f32_to_16<DT>(o[3])};
                            *reinterpret_cast<u32x2*>(orow + 16 * db + 4 * G) = __builtin_bit_cast(u32x2, h4);
                        }
                        if (G == 0) {
                            int64_t li_off = a.cu_seqlens_q ? (int64_t)h * a.lse_sh + a.cu_seqlens_q[b] + i
                                                            : (int64_t)b * a.lse_sb + (int64_t)h * a.lse_sh + i;
                            a.lse[li_off] = lse;
                        }
                    } else {
                        const int64_t prow = (int64_t)w * BM + (r - tile_row0);
#pragma unroll
                        for (int db = 0; db < DBLK; ++db) {
                            *reinterpret_cast<f32x4*>(a.part_o + prow * D + 16 * db + 4 * G) = oacc[rb][db] * inv;
                        }
                        if (G == 0) a.part_lse[prow] = lse;
                    }
                }
            }
        } else {
            // WK > 1: WR == 1, RB == 1 -> 16 rows; merge the NW key-split states.
            float* s_o = reinterpret_cast<float*>(s_raw);
            float* s_ml = s_o + C::NW * 16 * (D + 4);
            const float lrow = wave_sum16x4(l_run[0]);
            __syncthreads();  // every wave is done reading the K/V tile
            if (G == 0) {
                s_ml[(wave * 16 + li) * 2] = m_run[0];
                s_ml[(wave * 16 + li) * 2 + 1] = lrow;
            }
            __syncthreads();
            float mstar = -INFINITY;
#pragma unroll
            for (int v = 0; v < C::NW; ++v) mstar = fmaxf(mstar, s_ml[(v * 16 + li) * 2]);
            float L = 0.f;
#pragma unroll
            for (int v = 0; v < C::NW; ++v) {
                float mv = s_ml[(v * 16 + li) * 2];
                L += (mv == -INFINITY ? 0.f : fast_exp2(mv - mstar)) * s_ml[(v * 16 + li) * 2 + 1];
            }
            const float f = (m_run[0] == -INFINITY || !(L > 0.f)) ? 0.f : fast_exp2(m_run[0] - mstar) / L;
#pragma unroll
            for (int db = 0; db < DBLK; ++db)
                *reinterpret_cast<f32x4*>(s_o + (wave * 16 + li) * (D + 4) + 16 * db + 4 * G) = oacc[0][db] * f;
            __syncthreads();
            for (int idx = tid; idx < 16 * DCH; idx += NT) {
                const int rr = idx / DCH, d0 = (idx % DCH) * 8;
                const int r = tile_row0 + rr;
                if (rr >= tile_rows) continue;
                f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int v = 0; v < C::NW; ++v) {
                    acc0 += *reinterpret_cast<const f32x4*>(s_o + (v * 16 + rr) * (D + 4) + d0);
                    acc1 += *reinterpret_cast<const f32x4*>(s_o + (v * 16 + rr) * (D + 4) + d0 + 4);
                }
                float ms = -INFINITY, Ls = 0.f;
#pragma unroll
                for (int v = 0; v < C::NW; ++v) ms = fmaxf(ms, s_ml[(v * 16 + rr) * 2]);
#pragma unroll
                for (int v = 0; v < C::NW; ++v) {
                    float mv = s_ml[(v * 16 + rr) * 2];
                    Ls += (mv == -INFINITY ? 0.f : fast_exp2(mv - ms)) * s_ml[(v * 16 + rr) * 2 + 1];
                }
                const bool nonempty = Ls > 0.f;
                const float lse = nonempty ? (ms + fast_log2(Ls)) * kLn2 : (final_out ? INFINITY : -INFINITY);
                const int i = r / g, h = hk * g + r % g;
                if (final_out) {
                    uint16_t* orow;
                    if (a.cu_seqlens_q) orow = op + ((int64_t)a.cu_seqlens_q[b] + i) * a.o_si + (int64_t)h * a.o_sh;
                    else orow = op + (int64_t)b * a.o_sb + (int64_t)i * a.o_si + (int64_t)h * a.o_sh;
                    uint16_t h8[8] = {f32_to_16<DT>(acc0[0]), f32_to_16<DT>(acc0[1]), f32_to_16<DT>(acc0[2]),
                                      f32_to_16<DT>(acc0[3]), f32_to_16<DT>(acc1[0]), f32_to_16<DT>(acc1[1]),
                                      f32_to_16<DT>(acc1[2]), f32_to_16<DT>(acc1[3])};
                    *reinterpret_cast<u32x4*>(orow + d0) = __builtin_bit_cast(u32x4, h8);
                    if (d0 == 0) {
                        int64_t lo_off = a.cu_seqlens_q ? (int64_t)h * a.lse_sh + a.cu_seqlens_q[b] + i
                                                        : (int64_t)b * a.lse_sb + (int64_t)h * a.lse_sh + i;
                        a.lse[lo_off] = lse;
                    }
                } else {
                    const int64_t prow = (int64_t)w * BM + rr;
                    *reinterpret_cast<f32x4*>(a.part_o + prow * D + d0) = acc0;
                    *reinterpret_cast<f32x4*>(a.part_o + prow * D + d0 + 4) = acc1;
                    if (d0 == 0) a.part_lse[prow] = lse;
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
    *reinterpret_cast<u32x4*>(orow + d0) = __builtin_bit_cast(u32x4, h8);
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

// prefill: 128-row tile per item, 4 waves x 32 rows share each 64-key tile
template <int DT, int D> using PrefillCfg = Cfg<DT, D, 4, 1, 2, 64, 2>;

template <class C>
static hipError_t launch_fwd_cfg(const FwdArgs& a, int grid, hipStream_t stream) {
    hipLaunchKernelGGL(fa_fwd_kernel<C>, dim3(grid), dim3(C::NT), 0, stream, a);
    return hipGetLastError();
}


}  // namespace fa

// Exposed to fa_api.cpp (C++ linkage inside the library).
namespace fa {
int fwd_tile_rows() { return PrefillCfg<DT_BF16, 128>::BM; }
int fwd_tile_keys() { return PrefillCfg<DT_BF16, 128>::BN; }

hipError_t launch_fwd(const FwdArgs& a, int dtype, int d, int grid, hipStream_t stream) {
    if (d != 128) return hipErrorInvalidValue;
    return dtype == DT_BF16 ? launch_fwd_cfg<PrefillCfg<DT_BF16, 128>>(a, grid, stream)
                            : launch_fwd_cfg<PrefillCfg<DT_FP16, 128>>(a, grid, stream);
}

hipError_t launch_merge(const FwdArgs& a, int dtype, int d, hipStream_t stream) {
    if (d != 128) return hipErrorInvalidValue;
    const int64_t grid = (int64_t)a.B * a.mt_max * a.Hk * (128 / 16);
    if (dtype == DT_BF16) hipLaunchKernelGGL((fa_merge_kernel<DT_BF16, 128, 128>), dim3(grid), dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((fa_merge_kernel<DT_FP16, 128, 128>), dim3(grid), dim3(256), 0, stream, a);
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
