// Host check of the decode split (flash-attention-npu_amd/csrc/fa_decode_split.h)
// against brute force: for random sequence / kv-head / worker counts, with empty
// sequences among them, every tile belongs to exactly one worker; the owner
// the merge computes from a tile's cost is the worker whose range the kernel's
// split_tfirst gives that tile; when T >= W the workers between a segment's
// first and last owner each own a tile of it; and the merge's test for "the
// first owner also owns the tile before the segment" is what the ranges say.
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "fa_decode_split.h"

using namespace fa::dec;

static int failures = 0;
#define CHECK(cond, ...)                                  \
    do {                                                  \
        if (!(cond)) {                                    \
            if (++failures <= 20) {                       \
                std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
                std::printf(__VA_ARGS__);                 \
                std::printf("\n");                        \
            }                                             \
        }                                                 \
    } while (0)

static void check_case(const std::vector<int>& nts, int Hk, long long W, long long ovh_forced) {
    const int B = (int)nts.size();
    std::vector<int> pref(B + 1, 0);
    for (int b = 0; b < B; ++b) pref[b + 1] = pref[b] + Hk * nts[b];
    const long long T = pref[B];
    if (T == 0) return;
    const long long ovh = ovh_forced >= 0 ? ovh_forced : seg_ovh(T, W, (long long)B * Hk);
    const long long CT = split_total(T, ovh, B, Hk);
    // brute force: each tile's segment and cost
    std::vector<long long> cost(T), seg(T);
    for (int b = 0; b < B; ++b)
        for (int hk = 0; hk < Hk; ++hk)
            for (int i = 0; i < nts[b]; ++i) {
                const long long t = pref[b] + (long long)hk * nts[b] + i;
                seg[t] = (long long)b * Hk + hk;
                cost[t] = t + ovh * seg[t];
            }
    // the kernel's ranges
    std::vector<int> start(W + 1);
    for (long long w = 0; w <= W; ++w) start[w] = split_tfirst(w * CT / W, pref.data(), B, Hk, ovh, T, CT);
    CHECK(start[0] == 0 && start[W] == T, "ends T=%lld W=%lld", T, W);
    std::vector<long long> own(T, -1);
    for (long long w = 0; w < W; ++w) {
        CHECK(start[w] <= start[w + 1], "order w=%lld", w);
        for (int t = start[w]; t < start[w + 1]; ++t) own[t] = w;
    }
    for (long long t = 0; t < T; ++t) {
        CHECK(own[t] >= 0, "unowned tile %lld", t);
        // the merge's owner of a tile from its cost
        CHECK(split_owner(cost[t], W, CT) == own[t], "owner t=%lld cost=%lld got %lld want %lld", t, cost[t],
              split_owner(cost[t], W, CT), own[t]);
    }
    // per segment: the merge's worker list and the slot of its first partial
    for (int b = 0; b < B; ++b) {
        const int per = nts[b];
        if (per == 0) continue;
        for (int hk = 0; hk < Hk; ++hk) {
            const long long S = pref[b] + (long long)hk * per;
            const long long j = (long long)b * Hk + hk;
            const long long wf = split_owner(S + ovh * j, W, CT);
            const long long wl = split_owner(S + per - 1 + ovh * j, W, CT);
            if (T >= W)
                for (long long w = wf; w <= wl; ++w) {
                    bool has = false;
                    for (long long t = S; t < S + per; ++t) has = has || own[t] == w;
                    CHECK(has, "worker %lld between owners of segment (%d,%d) owns none of it", w, b, hk);
                }
            if (S > 0) {
                const long long jp = ovh > 0 ? split_prev_segment(b, hk, Hk, pref.data()) : 0;
                CHECK(ovh == 0 || seg[S - 1] == jp, "previous segment of (%d,%d): %lld want %lld", b, hk, jp, seg[S - 1]);
                const bool slot1 = split_owner(S - 1 + ovh * jp, W, CT) == wf;
                CHECK(slot1 == (start[wf] < S), "slot of segment (%d,%d)", b, hk);
            }
        }
    }
}

int main() {
    std::mt19937 rng(7);
    const int lens[] = {0, 0, 1, 2, 5, 17, 40, 90, 300};
    const long long Ws[] = {4, 16, 64, 1024};
    const int Hks[] = {1, 2, 8};
    int cases = 0;
    for (int it = 0; it < 600; ++it) {
        const int B = 1 + (int)(rng() % 64);
        const int Hk = Hks[rng() % 3];
        const long long W = Ws[rng() % 4];
        std::vector<int> nts(B);
        for (int& n : nts) n = lens[rng() % 9];
        check_case(nts, Hk, W, -1);  // the kernel's own choice of ovh
        long long T = 0;
        for (int n : nts) T += (long long)Hk * n;
        if (T >= 16 * W) {  // and the split by cost wherever it is allowed
            check_case(nts, Hk, W, 1);
            check_case(nts, Hk, W, 2);
        }
        ++cases;
    }
    // the config-3 shape: 64 sequences, 8 kv heads, 1024 workers
    {
        std::vector<int> nts(64);
        for (int b = 0; b < 64; ++b) nts[b] = 16 + (int)(rng() % 1000);
        check_case(nts, 8, 1024, -1);
        ++cases;
    }
    std::printf("%d cases, %d failures\n", cases, failures);
    return failures == 0 ? 0 : 1;
}
