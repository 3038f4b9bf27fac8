// fa_decode.hip -- decode attention for gfx950 (<= 16 packed query rows per kv
// head): KV-cache streaming at HBM speed.
//
// Same results as the reference forward (SplitFuse::FAInfer in flash-decode
// mode, csrc/arch22/flash_attn_npu_v2/mha_fwd_kvcache.cpp:250-316 with the
// CombineScale merge at :412-433 and CombineScale.hpp:76-357), organised for
// MI355X instead of the reference's per-core (B, N1, S1, S2) ranges
// (csrc/arch22/flash_attn_npu_v3/fa_split.h:483-510):
//   * The work list is every 32-key tile of every (sequence, kv head)
//     "segment", built in LDS from cache_seqlens by each workgroup (no host
//     round trip). The tiles are cut into equal contiguous ranges, one per
//     wave ("worker"), so uneven sequence lengths still balance exactly; the
//     waves of one CU share a range and stream adjacent kv heads of it when
//     the kv head count allows (4 heads per CU, else 2; dec_hs below).
//   * A worker streams its tiles with a STAGES-deep register pipeline of
//     16-byte loads (K straight into MFMA operand layout, V through a
//     wave-private LDS tile read back transposed), so each wave keeps up to
//     (STAGES-1) x 16 KB of HBM reads in flight without any block barrier.
//   * The g = H/Hk query heads of a kv head (x the query positions) form the
//     16 rows of one MFMA tile, so every cache byte is read once per call.
//   * A segment owned entirely by one worker is written final; a segment cut
//     by worker boundaries leaves <= 2 fp32 partials per worker, merged by
//     fa_decode_merge_kernel (the kernel boundary orders the partials).
#include "fa_common.h"
#include "fa_kernel_args.h"
#include "fa_decode_split.h"

#include <type_traits>

namespace fa {
namespace dec {
constexpr int NWAVE = 4;     // waves (workers) per workgroup
constexpr int TABN = 256;    // paged: block ids staged per wave
constexpr int MAXB = 2048;
// merge workgroups per segment (each merges D / split dims): 4 where segments
// carry 8 or more partials on average (c5 shapes: 9.5 us against 12.7 us with
// 2), else 2 (c2: 8.1 against 9.1 us; one box, bench stage events)
constexpr int MERGE_SPLIT_MANY = 4, MERGE_SPLIT_FEW = 2;

}  // namespace dec

#ifdef FA_DECODE_PHASES
// Instrumented build only (libfa_mi355x_phases.so, never the product
// library): per-wave real-time stamps (s_memrealtime, 100 MHz) of the last
// decode launch, 8 words per wave: entry, end of the plan, end of the first
// tile, exit, segments, tiles, HW_ID, XCC_ID. bench.py --phases reads them.
constexpr int kPhaseWaves = 8192;
__device__ unsigned long long fa_phase_stamps[kPhaseWaves * 8];
#define FA_PHASE(...) __VA_ARGS__
#else
#define FA_PHASE(...)
#endif

// Tile shape per kernel head dim and stored element size EB: a tile is 16 KB
// of K and V (32 keys at head dim 128, 64 keys at 64), so a wave keeps the
// same bytes in flight and every lane loads full 16-byte chunks. FP8 tiles
// hold 64 keys at both head dims (16 KB at 128, 8 KB at 64): at 32 keys the
// tile's fixed latency chain (QK -> softmax -> PV, one wave per SIMD), not
// HBM, set the pace, and 128-key tiles at head dim 64 spill.
template <int HD, int EB = 2>
struct DecCfg {
    static constexpr int D = HD;
    static constexpr int KT = 8192 / (HD * EB) < 64 ? 8192 / (HD * EB) : 64;  // keys per tile
    static constexpr int NH = KT / 16;     // 16-key blocks per tile
    static constexpr int KSTEPS = D / 32;
    static constexpr int DBLK = D / 16;
    // 16-byte chunk swizzle of the wave's V tile (row-major, D / 8 chunks per row)
    static __device__ __forceinline__ int vswz(int r, int c) { return HD == 64 ? swz_v64(r, c) : (c ^ (r & 15)); }
};

// Heads per worker group: when the kv head count is a multiple of 4, the 4
// waves of a workgroup (one CU) stream kv heads 4g .. 4g + 3 of the same
// sequence over the same tile range, so the CU requests the 4 adjacent
// head pieces of each key row together (1 KiB for bf16 at head dim 128); with
// an even count that is not, waves 0, 1 and 2, 3 form such groups of 2.
// Measured (one box, alternating runs, attention us): one head per wave ->
// pairs, c2 118.4-119.3 -> 116.3, c3 301.2-302.9 -> 297.0-297.6, c5 39.7-40.2
// -> 39.1-39.2, c3f8 unchanged; pairs -> 4 heads, c2 119.0-119.5 -> 115.4-115.9,
// c3 297.8-298.3 -> 295.2-295.5, c5 39.3-39.5 -> 39.4-39.8, c3f8 172.9-173.0 ->
// 173.5-173.7.
// The tile list and the split then run over head groups: group g of sequence b
// holds that sequence's tiles once, each wave of the group takes its head.
__device__ __forceinline__ int dec_hs(const FwdArgs& a) { return (a.Hk % 4) == 0 ? 4 : ((a.Hk % 2) == 0 ? 2 : 1); }

struct DecSeg {
    int S, n;         // first global tile, tiles
    int b, hk;
    int kvh;          // kv head of the segment's row tile (hk, or hk / kvdiv unpacked)
    int lo_tile;      // first 32-key tile of the sequence's visible key range
    int sk, sq, crow;
    int lp;           // cache_leftpad: key j is cache row lp + j (contiguous caches)
    int nf;           // key index of this call's first new token (cache_seqlens - lp)
};

// Per-batch facts kept in LDS: first tile, key count, query count, cache row.
struct DecBatch {
    int lo_tile, sk, sq, crow, lp, nf;
};

template <int KT>
__device__ __forceinline__ void dec_batch(const FwdArgs& a, int b, DecBatch& d, int& ntiles) {
    int sq = a.cu_seqlens_q ? a.cu_seqlens_q[b + 1] - a.cu_seqlens_q[b] : a.Sq;
    int sk;
    const int lp = a.leftpad ? min(max(a.leftpad[b], 0), a.kv_capacity) : 0;
    // new tokens sit at keys nf .. nf + seqlen_new - 1; those beyond the
    // capacity are neither attended nor written (sk is clamped below)
    d.nf = a.seqlens_k ? a.seqlens_k[b] - lp : 0;
    if (a.seqlens_k) sk = a.seqlens_k[b] + (a.cu_knew ? a.cu_knew[b + 1] - a.cu_knew[b] : a.seqlen_new) - lp;
    else if (a.cu_seqlens_k) sk = a.cu_seqlens_k[b + 1] - a.cu_seqlens_k[b];
    else sk = a.Sk;
    sq = min(max(sq, 0), a.Sq);
    sk = min(max(sk, 0), a.kv_capacity - lp);
    const int lo = max(0, key_lo(sk - sq, a.wl, a.chunk));
    const int hi = min(sk, key_hi(sk - 1, a.wr, a.chunk) + 1);
    d.lp = lp;
    d.sq = sq;
    d.sk = sk;
    d.lo_tile = lo / KT;
    const int bt_rows_or_cache = a.block_table ? a.bt_rows : a.batch_cache;
    d.crow = a.batch_idx ? min(max(a.batch_idx[b], 0), bt_rows_or_cache - 1) : b;
    ntiles = (sq > 0 && hi > lo) ? (hi + KT - 1) / KT - d.lo_tile : 0;
}

// segment of group tile t for head h of the group (hs heads per group)
__device__ __forceinline__ DecSeg dec_seg_of(const FwdArgs& a, const int* s_pref, const DecBatch* s_b, int t, int hs,
                                             int h) {
    int bl = 0, bh = a.B;
    while (bh - bl > 1) {
        int mid = (bl + bh) >> 1;
        if (s_pref[mid] <= t) bl = mid; else bh = mid;
    }
    DecSeg s;
    s.b = bl;
    const int per = (s_pref[bl + 1] - s_pref[bl]) / (a.Hk / hs);
    s.n = per;
    const int o = t - s_pref[bl];
    const int hg = per > 0 ? o / per : 0;
    s.hk = hg * hs + h;
    s.S = s_pref[bl] + hg * per;
    s.kvh = a.kvdiv == 1 ? s.hk : s.hk / a.kvdiv;
    const DecBatch d = s_b[bl];
    s.lo_tile = d.lo_tile;
    s.sk = d.sk;
    s.sq = d.sq;
    s.crow = d.crow;
    s.lp = d.lp;
    s.nf = d.nf;
    return s;
}

// BIAS: softcap or ALiBi present; FUSE: append k_new/v_new in this kernel;
// LAYOUT: 0 = batch-strided cache, 1 = paged with page % 32 == 0, 2 = any;
// HDM: head dim below 128 (dims >= a.hd read as zero, never written).
// QV: the scores add qv . v (one more MFMA chain per 16 keys, V against the
// qv row, into the same accumulator); 16-bit inputs only.
// DT_FP8: the cache, q and k_new / v_new hold e4m3fn bytes. The register
// pipeline carries the raw bytes (half the registers and half the HBM bytes
// of a bf16 cache). S^T = K.Q^T runs as 16x16x128 e4m3 MFMAs on those bytes;
// V is widened to bf16 on its way into the wave's LDS tile, and P.V stays a
// bf16 product. The descales scale the scores (q_descale * k_descale) and
// the output (v_descale).
template <int DT, int HD, int STAGES, bool BIAS, bool FUSE, int LAYOUT, bool HDM = false, bool QV = false>
__global__ void __launch_bounds__(256, 1) fa_decode_kernel(FwdArgs a) {
    using namespace dec;
    constexpr bool F8 = DT == DT_FP8;
    static_assert(!(QV && F8), "qv takes 16-bit inputs");
    using C = DecCfg<HD, F8 ? 1 : 2>;
    constexpr int D = C::D, KT = C::KT, NH = C::NH, KSTEPS = C::KSTEPS, DBLK = C::DBLK;
    using ET = std::conditional_t<F8, uint8_t, uint16_t>;  // stored element
    constexpr int EPL = 16 / sizeof(ET);                    // elements per 16-byte load
    constexpr int KL = F8 ? KSTEPS / 2 : KSTEPS;            // 16-byte loads per lane and key row
    __shared__ int s_pref[MAXB + 1];
    __shared__ DecBatch s_bat[MAXB];
    __shared__ int s_tab[NWAVE][TABN];
    __shared__ __attribute__((aligned(16))) uint16_t s_v[NWAVE][KT * D];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, G = lane >> 4;
    // 8-dim chunk of the head dim that lane group G holds in MFMA step s: for
    // bf16 / fp16 chunk 4s + G, so one 16-byte load instruction covers 64
    // contiguous bytes of each of its 16 key rows (the 4 lane groups side by
    // side); FP8 lane groups hold a quarter row each (the e4m3 MFMA's layout)
    auto chunk = [&](int s) -> int { return F8 ? G * KSTEPS + s : 4 * s + G; };
    // element offset, within a key row, of 16-byte load s of lane group G
    auto loff = [&](int s) -> int { return F8 ? G * (D / 4) + s * EPL : 8 * chunk(s); };
    FA_PHASE(const unsigned long long ph_entry = __builtin_amdgcn_s_memrealtime();
             unsigned long long ph_plan = 0, ph_first = 0, ph_nseg = 0;
             auto ph_write = [&](long long w, long long ntiles) {
                 if (lane == 0 && w < kPhaseWaves) {
                     unsigned long long* o = fa_phase_stamps + w * 8;
                     o[0] = ph_entry; o[1] = ph_plan; o[2] = ph_first;
                     o[3] = __builtin_amdgcn_s_memrealtime(); o[4] = ph_nseg; o[5] = (unsigned long long)ntiles;
                     o[6] = (unsigned)__builtin_amdgcn_s_getreg((31 << 11) | 4);   // HW_ID
                     o[7] = (unsigned)__builtin_amdgcn_s_getreg((15 << 11) | 20);  // XCC_ID
                 }
             };)

    // ---- plan: tiles per segment, prefix over batches -------------------------------
    for (int b = tid; b < a.B; b += 256) {
        DecBatch d;
        int nt;
        dec_batch<KT>(a, b, d, nt);
        s_bat[b] = d;
        s_pref[b + 1] = (a.Hk / dec_hs(a)) * nt;
    }
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
    if (blockIdx.x == 0)
        for (int b = tid; b <= a.B; b += 256) a.sched[b] = s_pref[b];

    const long long T = s_pref[a.B];
    const int hs = dec_hs(a), hgs = a.Hk / hs;  // heads per group, groups per sequence
    const int hsel = wave % hs;                   // this wave's head within its group
    const long long W = (long long)gridDim.x * (NWAVE / hs);  // group workers
    // workers are numbered wave-major: the 4 waves of a CU take tile ranges a
    // quarter of the tile list apart instead of 4 neighbouring ones, so they
    // do not stream neighbouring addresses of one (sequence, kv head) at the
    // same time (c2 attention 124.0 -> 120.4 us, c3 319.7 -> 312.4 us, c2f8
    // 76.6 -> 72.1 us on one box)
    const long long gw = (long long)(wave / hs) * gridDim.x + blockIdx.x;
    const long long wid = gw * hs + hsel;  // this wave's partial slots
    // tiles [t0, t1) of this worker: the split by cost of fa_decode_split.h
    const long long ovh = seg_ovh(T, W, (long long)a.B * hgs);
    const long long CT = split_total(T, ovh, a.B, hgs);
    const int t0 = split_tfirst(gw * CT / W, s_pref, a.B, hgs, ovh, T, CT);
    const int t1 = split_tfirst((gw + 1) * CT / W, s_pref, a.B, hgs, ovh, T, CT);
    FA_PHASE(ph_plan = __builtin_amdgcn_s_memrealtime(); if (t0 >= t1) ph_write(wid, 0);)
    if (t0 >= t1) return;  // no block barrier follows: waves are independent from here

    const ET* qp = static_cast<const ET*>(a.q);
    const ET* kp = static_cast<const ET*>(a.k);
    const ET* vp = static_cast<const ET*>(a.v);
    uint16_t* sv = s_v[wave];
    int* tab = s_tab[wave];
    const bool paged = LAYOUT == 1 || (LAYOUT == 2 && a.block_table != nullptr);
    const bool tab_ok = LAYOUT == 1;
    int tab_base = t0;

    auto fill_tab = [&](int base) {
        for (int i = lane; i < TABN; i += 64) {
            const int t = base + i;
            int blk = 0;
            if (t < t1) {
                DecSeg s = dec_seg_of(a, s_pref, s_bat, t, hs, hsel);
                const int key0 = (s.lo_tile + (t - s.S)) * KT;
                const int pidx = a.page_shift >= 0 ? key0 >> a.page_shift : key0 / a.page;
                blk = a.block_table[(int64_t)s.crow * a.bt_stride + pidx];
                blk = min(max(blk, 0), a.num_blocks - 1);
            }
            tab[i] = blk;
        }
    };
    if (tab_ok) fill_tab(tab_base);

    // ---- issue side: STAGES-deep register pipeline ------------------------------------
    u32x4 kr[STAGES][NH][KL], vr[STAGES][NH][KL];
    int bk[STAGES];  // paged block id of each in-flight tile
    DecSeg is = dec_seg_of(a, s_pref, s_bat, t0, hs, hsel);

    auto row_ptr = [&](const ET* base, int64_t sb, int64_t si, int64_t sh, const DecSeg& s, int key,
                       int blk) -> const ET* {
        if (paged) {
            int b2 = blk;
            if (!tab_ok) {
                const int pidx = key / a.page;
                b2 = min(max(a.block_table[(int64_t)s.crow * a.bt_stride + pidx], 0), a.num_blocks - 1);
            }
            const int inpage = a.page_shift >= 0 ? (key & (a.page - 1)) : key % a.page;
            return base + (int64_t)b2 * sb + (int64_t)inpage * si + (int64_t)s.kvh * sh;
        }
        if (LAYOUT == 2 && a.cu_seqlens_k)
            return base + ((int64_t)a.cu_seqlens_k[s.b] + key) * si + (int64_t)s.kvh * sh;
        return base + (int64_t)s.crow * sb + (int64_t)(s.lp + key) * si + (int64_t)s.kvh * sh;
    };

    // With a fused append, keys nf .. sk - 1 come from k_new / v_new; the
    // worker that owns their tile also writes them into the cache (each tile
    // has exactly one owner, and no other tile reads those positions). New
    // tokens past the cache capacity (nf + seqlen_new > sk) are dropped, as
    // the separate append kernel drops them.
    constexpr bool fuse = FUSE;
    const ET* knp = static_cast<const ET*>(a.k_new);
    const ET* vnp = static_cast<const ET*>(a.v_new);

    auto issue = [&](int t, u32x4 (&kk)[NH][KL], u32x4 (&vv)[NH][KL], int& blk) {
        if (t >= t1) return;
        if (t >= is.S + is.n) is = dec_seg_of(a, s_pref, s_bat, t, hs, hsel);
        blk = 0;
        if (tab_ok) {
            if (t >= tab_base + TABN) {
                tab_base += TABN;
                fill_tab(tab_base);
            }
            blk = tab[t - tab_base];
        }
        const int key0 = (is.lo_tile + (t - is.S)) * KT;
        const int first_new = fuse ? is.nf : 0x7fffffff;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            const int key = key0 + h * 16 + li;
            if (key < is.sk) {
                const ET* kpr;
                const ET* vpr;
                if (key >= first_new) {
                    const int tn = key - first_new;
                    const int64_t kvh = is.kvh;
                    kpr = knp + (int64_t)is.b * a.kn_sb + (int64_t)tn * a.kn_si + kvh * a.kn_sh;
                    vpr = vnp + (int64_t)is.b * a.vn_sb + (int64_t)tn * a.vn_si + kvh * a.vn_sh;
                } else {
                    kpr = row_ptr(kp, a.k_sb, a.k_si, a.k_sh, is, key, blk);
                    vpr = row_ptr(vp, a.v_sb, a.v_si, a.v_sh, is, key, blk);
                }
#pragma unroll
                for (int s = 0; s < KL; ++s) {
                    const bool in = !HDM || loff(s) < a.hd;
                    kk[h][s] = in ? *reinterpret_cast<const u32x4*>(kpr + loff(s)) : u32x4{0u, 0u, 0u, 0u};
                    vv[h][s] = in ? *reinterpret_cast<const u32x4*>(vpr + loff(s)) : u32x4{0u, 0u, 0u, 0u};
                }
            } else {
#pragma unroll
                for (int s = 0; s < KL; ++s) {
                    kk[h][s] = u32x4{0u, 0u, 0u, 0u};
                    vv[h][s] = u32x4{0u, 0u, 0u, 0u};
                }
            }
        }
    };

    // ---- compute side --------------------------------------------------------------------
    DecSeg cs = dec_seg_of(a, s_pref, s_bat, t0, hs, hsel);
    u32x4 qreg[KSTEPS];
    u32x4 qvreg[QV ? KSTEPS : 1];  // QV: the qv row
    u32x4 q8[2];  // FP8: the raw q bytes of dims G * D / 4 .. + D / 4 (zero-padded to 32)
    float slope = 0.f;
    int qi = 0;
    f32x4 oacc[DBLK];
    float m_run, l_run;
    int rows = 0;
    int seg_flo = 0, seg_fhi = 0;  // keys visible to every row of the segment: [seg_flo, seg_fhi]
    float sc_qk = a.scale, sc_qk2 = a.scale_log2, sc_v = 1.f;  // per segment (FP8 descales)

    auto begin_seg = [&](const DecSeg& s) {
        rows = s.sq * a.g;
        seg_flo = key_lo(s.sk - 1, a.wl, a.chunk);       // last row (diagonal sk - 1)
        seg_fhi = key_hi(s.sk - s.sq, a.wr, a.chunk);    // first row
        const bool ok = li < rows;
        const int i = ok ? li / a.g : 0;
        const int h = s.hk * a.g + (ok ? li % a.g : 0);
        qi = i;
        slope = (a.alibi && ok) ? a.alibi[(int64_t)s.b * a.alibi_sb + h] : 0.f;
        const ET* qrow = a.cu_seqlens_q
                             ? qp + ((int64_t)a.cu_seqlens_q[s.b] + i) * a.q_si + (int64_t)h * a.q_sh
                             : qp + (int64_t)s.b * a.q_sb + (int64_t)i * a.q_si + (int64_t)h * a.q_sh;
        if constexpr (F8) {
            // same bytes per lane as the K loads: B operand of the e4m3 MFMA
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const bool in = ok && s2 < KL && (!HDM || loff(s2) < a.hd);
                q8[s2] = in ? *reinterpret_cast<const u32x4*>(qrow + loff(s2)) : u32x4{0u, 0u, 0u, 0u};
            }
        } else {
#pragma unroll
            for (int s2 = 0; s2 < KSTEPS; ++s2) {
                const bool in = ok && (!HDM || 8 * chunk(s2) < a.hd);
                qreg[s2] = in ? *reinterpret_cast<const u32x4*>(qrow + 8 * chunk(s2)) : u32x4{0u, 0u, 0u, 0u};
            }
            if constexpr (QV) {
                // qv row of the same (position, head): B operand against V, as q against K
                const ET* qvp = static_cast<const ET*>(a.qv);
                const ET* qvrow = a.cu_seqlens_q
                                      ? qvp + ((int64_t)a.cu_seqlens_q[s.b] + i) * a.qv_si + (int64_t)h * a.qv_sh
                                      : qvp + (int64_t)s.b * a.qv_sb + (int64_t)i * a.qv_si + (int64_t)h * a.qv_sh;
#pragma unroll
                for (int s2 = 0; s2 < KSTEPS; ++s2) {
                    const bool in = ok && (!HDM || 8 * chunk(s2) < a.hd);
                    qvreg[s2] = in ? *reinterpret_cast<const u32x4*>(qvrow + 8 * chunk(s2)) : u32x4{0u, 0u, 0u, 0u};
                }
            }
        }
        if constexpr (F8) {
            const int kvh = s.kvh;
            const float qk = descale_at(a.qd, a.qd_sb, a.qd_sh, s.b, kvh) * descale_at(a.kd, a.kd_sb, a.kd_sh, s.b, kvh);
            sc_qk = a.scale * qk;
            sc_qk2 = a.scale_log2 * qk;
            sc_v = descale_at(a.vd, a.vd_sb, a.vd_sh, s.b, kvh);
        }
        m_run = -INFINITY;
        l_run = 0.f;
#pragma unroll
        for (int db = 0; db < DBLK; ++db) oacc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    };

    // The partial of the worker's first segment, when the worker goes on to
    // other segments, is held in registers and stored when the worker ends:
    // no partial store then enters the memory queue while the worker streams
    // (c3 attention ~314 -> ~309 us with all partial stores removed, timing-only
    // variant; the first segment's is the one mid-stream).
    f32x4 dpo[DBLK];
    float dlse = 0.f;
    int64_t dprow = -1;
    // Likewise the output of the latest whole segment: stored when the next
    // whole segment ends or when the worker ends.
    u32x2 hwo[DBLK];
    float hwlse = 0.f;
    uint16_t* hworow = nullptr;
    int64_t hwoff = -1;
    auto flush_whole = [&]() {
        if (hworow == nullptr) return;
#pragma unroll
        for (int db = 0; db < DBLK; ++db) {
            if (HDM && 16 * db + 4 * G >= a.hd) continue;
            *reinterpret_cast<u32x2*>(hworow + 16 * db + 4 * G) = hwo[db];
        }
        if (G == 0) a.lse[hwoff] = hwlse;
        hworow = nullptr;
    };

    auto end_seg = [&](const DecSeg& s) {
        const float lrow = wave_sum16x4(l_run);
        const bool nonempty = lrow > 0.f;
        const float inv = nonempty ? (F8 ? sc_v / lrow : 1.f / lrow) : 0.f;
        const bool whole = s.S >= t0 && s.S + s.n <= t1;
        if (li >= rows) return;
        if (whole) {
            const int i = li / a.g, h = s.hk * a.g + li % a.g;
            uint16_t* op = static_cast<uint16_t*>(a.out);
            uint16_t* orow = a.cu_seqlens_q
                                 ? op + ((int64_t)a.cu_seqlens_q[s.b] + i) * a.o_si + (int64_t)h * a.o_sh
                                 : op + (int64_t)s.b * a.o_sb + (int64_t)i * a.o_si + (int64_t)h * a.o_sh;
            flush_whole();
#pragma unroll
            for (int db = 0; db < DBLK; ++db) {
                f32x4 o = oacc[db] * inv;
                uint16_t h4[4] = {f32_to_16<DT>(o[0]), f32_to_16<DT>(o[1]), f32_to_16<DT>(o[2]), f32_to_16<DT>(o[3])};
                hwo[db] = __builtin_bit_cast(u32x2, h4);
            }
            hworow = orow;
            hwoff = a.cu_seqlens_q ? (int64_t)h * a.lse_sh + a.cu_seqlens_q[s.b] + i
                                   : (int64_t)s.b * a.lse_sb + (int64_t)h * a.lse_sh + i;
            hwlse = nonempty ? (m_run + fast_log2(lrow)) * kLn2 : INFINITY;
        } else {
            const int slot = (s.S <= t0) ? 0 : 1;  // first segment of this worker, else its last
            const int64_t prow = (wid * 2 + slot) * 16 + li;
            const float plse = nonempty ? (m_run + fast_log2(lrow)) * kLn2 : -INFINITY;
            if (slot == 0 && s.S + s.n < t1) {  // more segments follow: store at the end
#pragma unroll
                for (int db = 0; db < DBLK; ++db) dpo[db] = oacc[db] * inv;
                dlse = plse;
                dprow = prow;
                return;
            }
#pragma unroll
            for (int db = 0; db < DBLK; ++db)
                *reinterpret_cast<f32x4*>(a.part_o + prow * D + 16 * db + 4 * G) = oacc[db] * inv;
            if (G == 0) a.part_lse[prow] = plse;
        }
    };

    auto compute = [&](int t, const u32x4 (&kk)[NH][KL], const u32x4 (&vv)[NH][KL], int blk) {
        const int key0 = (cs.lo_tile + (t - cs.S)) * KT;
        if (fuse && key0 + KT > cs.nf) {
            // this tile holds appended tokens: write them into the cache
            const int first_new = cs.nf;
            ET* kc = const_cast<ET*>(kp);
            ET* vc = const_cast<ET*>(vp);
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const int key = key0 + h * 16 + li;
                if (key >= first_new && key < cs.sk) {
                    ET* kd = const_cast<ET*>(row_ptr(kc, a.k_sb, a.k_si, a.k_sh, cs, key, blk));
                    ET* vd = const_cast<ET*>(row_ptr(vc, a.v_sb, a.v_si, a.v_sh, cs, key, blk));
#pragma unroll
                    for (int s = 0; s < KL; ++s) {
                        if (!HDM || loff(s) < a.hd) {
                            *reinterpret_cast<u32x4*>(kd + loff(s)) = kk[h][s];
                            *reinterpret_cast<u32x4*>(vd + loff(s)) = vv[h][s];
                        }
                    }
                }
            }
        }
        // 16-byte bf16 / fp16 operand s of key block h (FP8: half of a raw load, widened)
        auto opnd = [&](const u32x4 (&x)[NH][KL], int h, int s) -> u32x4 {
            if constexpr (F8) {
                const u32x4 r = x[h][s >> 1];
                return fp8x8_to_bf16((s & 1) ? u32x2{r[2], r[3]} : u32x2{r[0], r[1]});
            } else {
                return x[h][s];
            }
        };
        // V tile -> wave-private LDS (row-major, 16-byte XOR swizzle)
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            const int kl = h * 16 + li;
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) {
                const int ch = chunk(s);
                *reinterpret_cast<u32x4*>(sv + kl * D + (C::vswz(kl, ch) << 3)) = opnd(vv, h, s);
            }
        }
        // S^T = K . Q^T
        f32x4 sacc[NH];
#pragma unroll
        for (int h = 0; h < NH; ++h) sacc[h] = f32x4{0.f, 0.f, 0.f, 0.f};
        if constexpr (F8) {
            // one e4m3 MFMA per 16 keys over all dims: lane (li, G) holds key
            // li's and row li's dims G * D / 4 .. + D / 4, its raw loads (at
            // head dim 64 the upper 16 bytes are zero on both sides)
#pragma unroll
            for (int h = 0; h < NH; ++h)
                sacc[h] = mfma16x16x128_e4m3(kk[h][0], KL > 1 ? kk[h][KL - 1] : u32x4{0u, 0u, 0u, 0u}, q8[0], q8[1],
                                             sacc[h]);
        } else {
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
                for (int h = 0; h < NH; ++h) sacc[h] = mfma16x16x32<DT>(opnd(kk, h, s), qreg[s], sacc[h]);
            if constexpr (QV) {
                // S^T += V . Qv^T: the V loads carry the same lane layout as the K loads
#pragma unroll
                for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
                    for (int h = 0; h < NH; ++h) sacc[h] = mfma16x16x32<DT>(opnd(vv, h, s), qvreg[s], sacc[h]);
            }
        }
        // online softmax (log2 domain), row = li, keys key0 + 16h + 4G + e
        const int sk = cs.sk, diag0 = cs.sk - cs.sq;
        const bool full = key0 + KT <= sk && key0 >= seg_flo && key0 + KT - 1 <= seg_fhi;
        constexpr bool plain = !BIAS;
        float x[NH][4];
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float sv2 = sacc[h][e];
                float xv;
                if (plain) {
                    xv = sv2 * (F8 ? sc_qk2 : a.scale_log2);
                } else {
                    float y = sv2 * (F8 ? sc_qk : a.scale);
                    if (a.softcap > 0.f) y = a.softcap * fast_tanh(y * (1.f / a.softcap));
                    if (a.alibi) {
                        int dist = qi + diag0 - (key0 + h * 16 + G * 4 + e);
                        dist = dist < 0 ? -dist : dist;
                        y -= slope * (float)dist;
                    }
                    xv = y * kLog2e;
                }
                x[h][e] = xv;
            }
        if (!full) {
            const int dg = qi + diag0;
            const int rlo = key_lo(dg, a.wl, a.chunk), rhi = key_hi(dg, a.wr, a.chunk);
#pragma unroll
            for (int h = 0; h < NH; ++h)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int j = key0 + h * 16 + G * 4 + e;
                    const bool vis = j < sk && j >= rlo && j <= rhi;
                    x[h][e] = vis ? x[h][e] : -INFINITY;
                }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int h = 0; h < NH; ++h) tmax = fmaxf(tmax, fmaxf(fmaxf(x[h][0], x[h][1]), fmaxf(x[h][2], x[h][3])));
        tmax = wave_max16x4(tmax);
        const float m_new = fmaxf(m_run, tmax);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = fast_exp2(m_run - m_use);
        m_run = m_new;
        float p[NH][4], psum = 0.f;
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                p[h][e] = fast_exp2(x[h][e] - m_use);
                psum += p[h][e];
            }
        l_run = l_run * alpha + psum;
        // P^T operands, one per 32 keys: blocks 2k and 2k + 1
        u32x4 pk[NH / 2];
#pragma unroll
        for (int k2 = 0; k2 < NH / 2; ++k2) {
            f32x8 p8 = {p[2 * k2][0], p[2 * k2][1], p[2 * k2][2], p[2 * k2][3],
                        p[2 * k2 + 1][0], p[2 * k2 + 1][1], p[2 * k2 + 1][2], p[2 * k2 + 1][3]};
            pk[k2] = pack8<DT>(p8);
        }
        // O^T += V^T . P^T with V^T from transpose reads of the LDS tile
        const int r4 = li >> 2, c4 = li & 3;
#pragma unroll
        for (int db = 0; db < DBLK; ++db) {
            const int ch = 2 * db + (c4 >> 1);
            const int off = (c4 & 1) * 4;
            f32x4 o = oacc[db] * alpha;
#pragma unroll
            for (int k2 = 0; k2 < NH / 2; ++k2) {
                const int ka = 32 * k2 + 4 * G + r4, kb = ka + 16;
                s16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(sv + ka * D + (C::vswz(ka, ch) << 3) + off));
                s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(sv + kb * D + (C::vswz(kb, ch) << 3) + off));
                u32x2 l2 = __builtin_bit_cast(u32x2, lo4);
                u32x2 h2 = __builtin_bit_cast(u32x2, hi4);
                u32x4 av = {l2[0], l2[1], h2[0], h2[1]};
                o = mfma16x16x32<DT>(av, pk[k2], o);
            }
            oacc[db] = o;
        }
    };

    // prologue: the first segment's q, then the first STAGES-1 tiles (loads
    // return in order, so q issued first is not held behind the K/V tiles)
    begin_seg(cs);
#pragma unroll
    for (int st = 0; st < STAGES - 1; ++st) issue(t0 + st, kr[st], vr[st], bk[st]);

    for (int tb = t0; tb < t1; tb += STAGES) {
#pragma unroll
        for (int st = 0; st < STAGES; ++st) {
            const int t = tb + st;
            if (t < t1) {
                issue(t + STAGES - 1, kr[(st + STAGES - 1) % STAGES], vr[(st + STAGES - 1) % STAGES],
                      bk[(st + STAGES - 1) % STAGES]);
                if (t >= cs.S + cs.n) {
                    end_seg(cs);
                    cs = dec_seg_of(a, s_pref, s_bat, t, hs, hsel);
                    begin_seg(cs);
                    FA_PHASE(++ph_nseg;)
                }
                compute(t, kr[st], vr[st], bk[st]);
                FA_PHASE(if (t == t0) ph_first = __builtin_amdgcn_s_memrealtime();)
            }
        }
    }
    end_seg(cs);
    flush_whole();
    if (dprow >= 0) {
#pragma unroll
        for (int db = 0; db < DBLK; ++db) *reinterpret_cast<f32x4*>(a.part_o + dprow * D + 16 * db + 4 * G) = dpo[db];
        if (G == 0) a.part_lse[dprow] = dlse;
    }
    FA_PHASE(++ph_nseg; ph_write(wid, t1 - t0);)
}

// Merge of the partials a segment left in the decode kernel (DSPLIT workgroups
// per segment, each on D / DSPLIT dims of the head; a segment with no visible key
// gets out = 0, lse = +inf): per row, lse = M + ln(sum_j exp(lse_j - M)) and
// O = sum_j exp(lse_j - lse) * O_j (the closed form of
// CombineScale.hpp:150-194). The partial list of a segment is known from the
// worker split alone: the tiles [S, S+n) of its kv head group belong to group
// workers owner(S)..owner(S+n-1) when every group worker has a tile (T >= W),
// else one group worker per tile, and within a group worker the wave of this
// kv head (hk % hs) wrote the head's partials. NG thread groups each
// fold a share of the partials in one pass with a running maximum (the lse
// and O of a partial are loaded together), and the groups are combined in
// LDS. (Merging inside the decode kernel, by the last wave to finish a
// segment, was measured 1.6x slower: every partial then needs a device-scope
// fence, i.e. an L2 write-back across the 8 XCDs.)
template <int DT, int D, int DSPLIT>
__global__ void __launch_bounds__(256) fa_decode_merge_kernel(FwdArgs a, int workers) {
    using namespace dec;
    __shared__ __attribute__((aligned(16))) float s_acc[256][8];
    __shared__ float s_gm[256], s_gs[256];
    constexpr int CH = D / DSPLIT / 8;   // 8-dim chunks per row in one workgroup
    const int sig = blockIdx.x / DSPLIT, dsl = blockIdx.x % DSPLIT;
    const int b = sig / a.Hk, hk = sig % a.Hk;
    const int hs = dec_hs(a), hgs = a.Hk / hs, hg = hk / hs, hsel = hk % hs;
    const long long sigg = (long long)b * hgs + hg;  // the segment's head group
    if (b >= a.B) return;
    int sq = a.cu_seqlens_q ? a.cu_seqlens_q[b + 1] - a.cu_seqlens_q[b] : a.Sq;
    sq = min(max(sq, 0), a.Sq);
    const int rows = sq * a.g;
    if (rows <= 0) return;
    const long long T = a.sched[a.B];
    const int per = (a.sched[b + 1] - a.sched[b]) / hgs;
    const long long S = a.sched[b] + (long long)hg * per;   // the group's first tile
    const long long W = workers / hs;                        // group workers
    const int tid = threadIdx.x;
    // the split of the decode kernel (fa_decode_split.h): tile t of segment j
    // costs t + ovh * j, and worker w owns the costs [w * CT / W, (w + 1) * CT / W)
    const long long ovh = seg_ovh(T, W, (long long)a.B * hgs);
    const long long CT = split_total(T, ovh, a.B, hgs);
    auto owner = [&](long long t) { return split_owner(t + ovh * sigg, W, CT); };  // t in this group
    long long wf = 0;
    int n = 0;
    if (per > 0) {
        wf = owner(S);
        n = T >= W ? (int)(owner(S + per - 1) - wf + 1) : per;
        if (n == 1) return;  // one worker owned the segment and wrote the result
    }
    // the first partial is its worker's second (slot 1) when that worker also
    // owns the tile before this segment; that tile's segment is the previous
    // one of this batch, else the last one of the nearest batch with tiles
    bool first_slot1 = false;
    if (per > 0 && S > 0) {
        // that tile's segment only matters through its cost, so only when ovh > 0
        const long long jp = ovh > 0 ? split_prev_segment(b, hg, hgs, a.sched) : 0;
        first_slot1 = split_owner(S - 1 + ovh * jp, W, CT) == wf;
    }
    // partial j of this segment -> its first partial row
    auto prow0 = [&](int j) -> long long {
        const long long w = T >= W ? wf + j : owner(S + j);
        const int slot = (j == 0 && first_slot1) ? 1 : 0;
        return ((w * hs + hsel) * 2 + slot) * 16;
    };
    // ---- one pass: each of NG thread groups folds its share of the partials
    // with a running maximum (lse and O of a partial are loaded together), then
    // the groups are combined through LDS ----------------------------------------------
    int rp = 1;
    while (rp < rows) rp <<= 1;
    const int GS = CH * rp;  // threads per group: one per (row, 8-dim chunk)
    const int NG = 256 / GS;
    const int grp = tid / GS, rem = tid % GS;
    const int rr = rem / CH, d0 = dsl * (D / DSPLIT) + (rem % CH) * 8;
    float m = -INFINITY, sum = 0.f;
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    if (rr < rows) {
#pragma unroll 4
        for (int j = grp; j < n; j += NG) {
            const long long pr = prow0(j) + rr;
            const float v = a.part_lse[pr];
            const f32x4 o0 = *reinterpret_cast<const f32x4*>(a.part_o + pr * D + d0);
            const f32x4 o1 = *reinterpret_cast<const f32x4*>(a.part_o + pr * D + d0 + 4);
            if (v != -INFINITY) {  // -inf: a partial that saw no key
                const float mn = fmaxf(m, v);
                const float c = fast_exp2((m - mn) * kLog2e), wgt = fast_exp2((v - mn) * kLog2e);
                acc0 = acc0 * c + o0 * wgt;
                acc1 = acc1 * c + o1 * wgt;
                sum = sum * c + wgt;
                m = mn;
            }
        }
    }
    if (NG > 1) {
        *reinterpret_cast<f32x4*>(&s_acc[tid][0]) = acc0;
        *reinterpret_cast<f32x4*>(&s_acc[tid][4]) = acc1;
        s_gm[tid] = m;
        s_gs[tid] = sum;
        __syncthreads();
        if (grp != 0) return;
        float M = m;
        for (int gq = 1; gq < NG; ++gq) M = fmaxf(M, s_gm[tid + gq * GS]);
        if (M != -INFINITY) {
            const float c = fast_exp2((m - M) * kLog2e);
            acc0 *= c;
            acc1 *= c;
            sum *= c;
            for (int gq = 1; gq < NG; ++gq) {
                const int o = tid + gq * GS;
                const float cg = fast_exp2((s_gm[o] - M) * kLog2e);  // 0 for an empty group
                acc0 += *reinterpret_cast<const f32x4*>(&s_acc[o][0]) * cg;
                acc1 += *reinterpret_cast<const f32x4*>(&s_acc[o][4]) * cg;
                sum += s_gs[o] * cg;
            }
        }
        m = M;
    }
    // lse of the row; -inf marks a row with no visible key (out = 0, lse = +inf)
    const float inv = m == -INFINITY ? 0.f : 1.f / sum;
    acc0 *= inv;
    acc1 *= inv;
    const float L = m == -INFINITY ? -INFINITY : m + fast_log2(sum) * kLn2;
    if (rr >= rows) return;
    const int i = rr / a.g, h = hk * a.g + rr % a.g;
    uint16_t* op = static_cast<uint16_t*>(a.out);
    uint16_t* orow = a.cu_seqlens_q ? op + ((int64_t)a.cu_seqlens_q[b] + i) * a.o_si + (int64_t)h * a.o_sh
                                    : op + (int64_t)b * a.o_sb + (int64_t)i * a.o_si + (int64_t)h * a.o_sh;
    uint16_t h8[8] = {f32_to_16<DT>(acc0[0]), f32_to_16<DT>(acc0[1]), f32_to_16<DT>(acc0[2]), f32_to_16<DT>(acc0[3]),
                      f32_to_16<DT>(acc1[0]), f32_to_16<DT>(acc1[1]), f32_to_16<DT>(acc1[2]), f32_to_16<DT>(acc1[3])};
    if (d0 < a.hd) *reinterpret_cast<u32x4*>(orow + d0) = __builtin_bit_cast(u32x4, h8);
    if (d0 == 0) {
        const int64_t off = a.cu_seqlens_q ? (int64_t)h * a.lse_sh + a.cu_seqlens_q[b] + i
                                           : (int64_t)b * a.lse_sb + (int64_t)h * a.lse_sh + i;
        a.lse[off] = L == -INFINITY ? INFINITY : L;
    }
}

constexpr int kDecodeStages = 3;
// FP8 tiles hold 64 keys (16 KB at head dim 128), so the bf16 depth keeps as
// many bytes in flight per wave
constexpr int kDecodeStagesF8 = 3;

int decode_workers(int cus) { return cus * dec::NWAVE; }

template <int DT, int HD, int LAYOUT>
static void launch_decode_l(const FwdArgs& a, int grid, hipStream_t stream) {
    const bool bias = a.softcap > 0.f || a.alibi != nullptr;
    const bool fuse = a.k_new != nullptr;
    constexpr int S = DT == DT_FP8 ? kDecodeStagesF8 : kDecodeStages;
    if (bias) {
        if (fuse) hipLaunchKernelGGL((fa_decode_kernel<DT, HD, S, true, true, LAYOUT>), dim3(grid), dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((fa_decode_kernel<DT, HD, S, true, false, LAYOUT>), dim3(grid), dim3(256), 0, stream, a);
    } else {
        if (fuse) hipLaunchKernelGGL((fa_decode_kernel<DT, HD, S, false, true, LAYOUT>), dim3(grid), dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((fa_decode_kernel<DT, HD, S, false, false, LAYOUT>), dim3(grid), dim3(256), 0, stream, a);
    }
}

template <int DT, int HD>
static void launch_decode_t(const FwdArgs& a, int grid, hipStream_t stream) {
    constexpr int KT = DecCfg<HD, DT == DT_FP8 ? 1 : 2>::KT;
    constexpr int S = DT == DT_FP8 ? kDecodeStagesF8 : kDecodeStages;
    if constexpr (DT != DT_FP8) {
        if (a.qv) {
            // qv: the generic-layout, bias-capable, dim-masking instances
            if (a.k_new) hipLaunchKernelGGL((fa_decode_kernel<DT, HD, S, true, true, 2, true, true>), dim3(grid), dim3(256), 0, stream, a);
            else hipLaunchKernelGGL((fa_decode_kernel<DT, HD, S, true, false, 2, true, true>), dim3(grid), dim3(256), 0, stream, a);
            return;
        }
    }
    if (a.hd < HD) {
        // head dims below the kernel's: the generic-layout, bias-capable
        // instances with dim masking (correct for every input of this kernel)
        if (a.k_new) hipLaunchKernelGGL((fa_decode_kernel<DT, HD, S, true, true, 2, true>), dim3(grid), dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((fa_decode_kernel<DT, HD, S, true, false, 2, true>), dim3(grid), dim3(256), 0, stream, a);
        return;
    }
    if (a.block_table && (a.page % KT) == 0) launch_decode_l<DT, HD, 1>(a, grid, stream);
    else if (a.block_table || a.cu_seqlens_k) launch_decode_l<DT, HD, 2>(a, grid, stream);
    else launch_decode_l<DT, HD, 0>(a, grid, stream);
}

// d: the kernel head dim, 64 or 128 (a.hd <= d is the head dim in memory)
hipError_t launch_decode(const FwdArgs& a, int dtype, int d, int grid, hipStream_t stream) {
    if (d != 64 && d != 128) return hipErrorInvalidValue;
    if (dtype == DT_BF16) {
        if (d == 64) launch_decode_t<DT_BF16, 64>(a, grid, stream);
        else launch_decode_t<DT_BF16, 128>(a, grid, stream);
    } else if (dtype == DT_FP8) {
        if (d == 64) launch_decode_t<DT_FP8, 64>(a, grid, stream);
        else launch_decode_t<DT_FP8, 128>(a, grid, stream);
    } else {
        if (d == 64) launch_decode_t<DT_FP16, 64>(a, grid, stream);
        else launch_decode_t<DT_FP16, 128>(a, grid, stream);
    }
    return hipGetLastError();
}

template <int DT, int DSPLIT>
static void launch_decode_merge_s(const FwdArgs& a, int d, int w, hipStream_t stream) {
    const int wgs = a.B * a.Hk * DSPLIT;  // DSPLIT workgroups per (sequence, kv head) segment
    if (d == 64) hipLaunchKernelGGL((fa_decode_merge_kernel<DT, 64, DSPLIT>), dim3(wgs), dim3(256), 0, stream, a, w);
    else hipLaunchKernelGGL((fa_decode_merge_kernel<DT, 128, DSPLIT>), dim3(wgs), dim3(256), 0, stream, a, w);
}

hipError_t launch_decode_merge(const FwdArgs& a, int dtype, int d, int grid, hipStream_t stream) {
    if (d != 64 && d != 128) return hipErrorInvalidValue;
    const int w = grid * dec::NWAVE;
    // partials per segment on average (every worker leaves at most 2)
    const bool many = (int64_t)w >= 8LL * a.B * a.Hk;
    const int odt = (dtype == DT_BF16 || dtype == DT_FP8) ? DT_BF16 : DT_FP16;  // FP8 inputs give a bf16 output
    if (odt == DT_BF16) {
        if (many) launch_decode_merge_s<DT_BF16, dec::MERGE_SPLIT_MANY>(a, d, w, stream);
        else launch_decode_merge_s<DT_BF16, dec::MERGE_SPLIT_FEW>(a, d, w, stream);
    } else {
        if (many) launch_decode_merge_s<DT_FP16, dec::MERGE_SPLIT_MANY>(a, d, w, stream);
        else launch_decode_merge_s<DT_FP16, dec::MERGE_SPLIT_FEW>(a, d, w, stream);
    }
    return hipGetLastError();
}

}  // namespace fa

#ifdef FA_DECODE_PHASES
// Device address and capacity (waves) of the stamp buffer of the instrumented build.
extern "C" __attribute__((visibility("default"))) int fa_decode_phase_stamps(void** ptr, int* waves) {
    *waves = fa::kPhaseWaves;
    return (int)hipGetSymbolAddress(ptr, HIP_SYMBOL(fa::fa_phase_stamps));
}
#endif
