// fa_decode_split.h -- the static split of the decode kernel's key tiles over
// its wave workers, shared by fa_decode_kernel (which tiles each worker
// streams), fa_decode_merge_kernel (which workers left partials of a segment)
// and the host check tests/host/fa_decode_split_check.cpp. Integer code only,
// callable from host and device.
//
// Tiles are numbered segment by segment: segment (b, hk) -- sequence b, kv
// head hk -- holds nt_b tiles starting at pref[b] + hk * nt_b, where pref[]
// is the tile prefix over the B sequences (pref[b + 1] - pref[b] = Hk * nt_b,
// pref[B] = T).
//
// The kernels call these functions with kv head GROUPS in place of kv heads:
// a group is 4 (or 2) adjacent heads streamed together by the 4 (or 2) waves
// of one CU, so Hk here is the group count and W the count of wave groups.
// The split itself does not depend on what a segment holds.
//
// Static split by cost: a worker that moves to another segment pays about a
// tile's time for it (the q reload and the store of the finished segment).
// Where workers cross many segments (at least half a segment per worker:
// B * Hk >= W / 2) and own at least 16 tiles each, every segment counts
// kSegCost tiles more, so workers crossing many short segments get fewer
// tiles. Tile t of segment j = b * Hk + hk costs t + ovh * j; worker w owns
// the tiles whose cost lies in [floor(w * CT / W), floor((w + 1) * CT / W)),
// CT = T + ovh * B * Hk. With ovh = 0 this is the plain split of T tiles.
// (Measured, one box, three runs each: c3 305.7 -> 303.8 us, c3f8 178.5 ->
// 175.3 us; c2, with a quarter segment per worker, was 2 us slower with it and
// keeps the plain split.)
#pragma once

#if defined(__HIPCC__) || defined(__HIP__)
#define FA_SPLIT_FN __host__ __device__ inline
#else
#define FA_SPLIT_FN inline
#endif

namespace fa {
namespace dec {

constexpr long long kSegCost = 1;

// the cost of a segment switch in tiles for T tiles, W workers, segs segments
FA_SPLIT_FN long long seg_ovh(long long T, long long W, long long segs) {
    return (T >= 16 * W && 2 * segs >= W) ? kSegCost : 0;
}

// the total cost CT
FA_SPLIT_FN long long split_total(long long T, long long ovh, int B, int Hk) { return T + ovh * B * Hk; }

// the first tile whose cost is >= c (T when none): segment starts in cost
// space are pref[b] + ovh * b * Hk for sequence b's first, then one every
// nt_b + ovh; a cost in the ovh-wide gap after a segment maps to the next
// segment's first tile
FA_SPLIT_FN int split_tfirst(long long c, const int* pref, int B, int Hk, long long ovh, long long T,
                             long long CT) {
    if (ovh == 0) return (int)c;
    if (c >= CT) return (int)T;
    // 32-bit arithmetic (a 64-bit division is a long instruction sequence on
    // the GPU): T counts 8-16 KB tiles, so CT = T + ovh * B * Hk stays far
    // below 2^31 for any cache that fits in memory
    const int ci = (int)c, ov = (int)ovh;
    int bl = 0, bh = B;
    while (bh - bl > 1) {
        const int mid = (bl + bh) >> 1;
        if (pref[mid] + ov * mid * Hk <= ci) bl = mid;
        else bh = mid;
    }
    const int cb = pref[bl] + ov * bl * Hk;
    const int nt = (pref[bl + 1] - pref[bl]) / Hk;
    int hk = (int)((unsigned)(ci - cb) / (unsigned)(nt + ov));
    if (hk > Hk - 1) hk = Hk - 1;
    int off = ci - cb - hk * (nt + ov);
    if (off > nt) off = nt;
    return pref[bl] + hk * nt + off;
}

// the worker whose cost range holds cost c (0 <= c < CT)
FA_SPLIT_FN long long split_owner(long long c, long long W, long long CT) { return ((c + 1) * W - 1) / CT; }

// the segment (b * Hk + hk) of the tile just before segment (b, hk)'s first
// tile, for a segment whose first tile is not tile 0: the previous kv head's
// segment of sequence b, else the last kv head's of the nearest earlier
// sequence that has tiles
FA_SPLIT_FN long long split_prev_segment(int b, int hk, int Hk, const int* pref) {
    if (hk > 0) return (long long)b * Hk + hk - 1;
    int bp = b - 1;
    while (bp > 0 && pref[bp + 1] == pref[bp]) --bp;
    return (long long)bp * Hk + Hk - 1;
}

}  // namespace dec
}  // namespace fa
