// Host-only harness for the C ABI's validation, planning and launch
// sequencing (flash-attention-npu_amd/csrc/fa_api.cpp), built with g++ and
// AddressSanitizer / UndefinedBehaviorSanitizer by tests/test_host_sanitize.py.
//
// The kernel launchers and the few HIP runtime calls fa_api.cpp makes are
// replaced here by recording stubs, so no GPU or HIP runtime is needed: each
// launch records its arguments, and the driver checks the invariants the
// kernels rely on (at most 2048 sequences per launch, every batch chunk
// covered once, pointers moved to the chunk's first sequence).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "fa_kernel_args.h"
#include "fa_mi355x.h"

// ---- HIP runtime stand-ins (host harness only) ---------------------------------------
extern "C" {
hipError_t hipGetDevice(int* d) {
    *d = 0;
    return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) {
    *v = 256;
    return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
const char* hipGetErrorString(hipError_t) { return "stub"; }
}

namespace {
struct Launch {
    char kind[16];
    int B;
    const void* q;
    const void* out;
    const float* lse;
    const int* seqlens;
};
std::vector<Launch> g_launch;
void rec(const char* k, int B, const void* q, const void* out, const float* lse, const int* sl) {
    Launch l{};
    snprintf(l.kind, sizeof(l.kind), "%s", k);
    l.B = B;
    l.q = q;
    l.out = out;
    l.lse = lse;
    l.seqlens = sl;
    g_launch.push_back(l);
}
}  // namespace

namespace fa {
int fwd_tile_rows(int d) { return d > 128 ? 128 : d > 64 ? 256 : 512; }
int fwd_tile_keys(int d) { return d > 128 ? 32 : 64; }
int decode_workers(int cus) { return cus * 4; }
int bwd_key_block(int d) { return d > 128 ? 64 : d > 64 ? 128 : 256; }
int bwd_row_block(int d) { return d > 128 ? 64 : 128; }
hipError_t launch_fwd(const FwdArgs& a, int, int, int, hipStream_t) {
    rec("fwd", a.B, a.q, a.out, a.lse, a.seqlens_k);
    return hipSuccess;
}
hipError_t launch_merge(const FwdArgs& a, int, int, hipStream_t) {
    rec("merge", a.B, a.q, a.out, a.lse, a.seqlens_k);
    return hipSuccess;
}
hipError_t launch_decode(const FwdArgs& a, int, int, int, hipStream_t) {
    rec("decode", a.B, a.q, a.out, a.lse, a.seqlens_k);
    return hipSuccess;
}
hipError_t launch_decode_merge(const FwdArgs& a, int, int, int, hipStream_t) {
    rec("dmerge", a.B, a.q, a.out, a.lse, a.seqlens_k);
    return hipSuccess;
}
hipError_t launch_combine_flat(const float*, const float*, int, int64_t, int, void*, int64_t, int, float*, hipStream_t) {
    rec("combine", 0, nullptr, nullptr, nullptr, nullptr);
    return hipSuccess;
}
hipError_t launch_kv_prep(const KvPrepArgs& a, int, hipStream_t) {
    rec("kvprep", a.B, a.q, nullptr, nullptr, a.seqlens);
    return hipSuccess;
}
hipError_t launch_bwd(const BwdArgs& a, int, int, int, int, hipStream_t) {
    rec("bwd", a.B, a.q, a.dq, a.lse, nullptr);
    return hipSuccess;
}
}  // namespace fa

static int g_fail = 0;
#define EXPECT(c, ...)                          \
    do {                                        \
        if (!(c)) {                             \
            fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);       \
            fprintf(stderr, "\n");              \
            ++g_fail;                           \
        }                                       \
    } while (0)

static fa_fwd_params base(int B, int Sq, int H, int Hk, int D, int cap) {
    fa_fwd_params p;
    memset(&p, 0, sizeof(p));
    p.abi_version = FA_MI355X_ABI_VERSION;
    p.dtype = FA_DTYPE_BF16;
    p.batch = B;
    p.seqlen_q = Sq;
    p.nheads = H;
    p.nheads_k = Hk;
    p.headdim = D;
    p.headdim_v = D;
    p.seqlen_k = cap;
    p.batch_cache = B;
    // fake, 16-byte aligned device addresses (never dereferenced by the host code)
    p.q = (const void*)0x100000;
    p.q_head_stride = D;
    p.q_row_stride = (int64_t)H * D;
    p.q_batch_stride = (int64_t)Sq * H * D;
    p.k = (void*)0x200000;
    p.v = (void*)0x300000;
    p.k_head_stride = p.v_head_stride = D;
    p.k_row_stride = p.v_row_stride = (int64_t)Hk * D;
    p.k_batch_stride = p.v_batch_stride = (int64_t)cap * Hk * D;
    p.out = (void*)0x400000;
    p.out_head_stride = D;
    p.out_row_stride = (int64_t)H * D;
    p.out_batch_stride = (int64_t)Sq * H * D;
    p.softmax_lse = (float*)0x500000;
    p.softmax_scale = 0.088f;
    p.is_causal = 1;
    p.window_size_left = -1;
    p.window_size_right = -1;
    return p;
}

// Runs `call` with a workspace of the size the library asks for and checks
// the chunking invariants of the recorded attention launches.
static void run_and_check(const char* what, fa_fwd_params p, int kind) {
    size_t ws = 0;
    fa_status_t st = fa_fwd_workspace_size(&p, kind, &ws);
    EXPECT(st == FA_OK, "%s: workspace_size -> %d (%s)", what, st, fa_last_error());
    if (st != FA_OK) return;
    std::vector<unsigned char> host(1);
    p.workspace = (void*)0x7000000000ull;  // 256-byte aligned fake device address
    p.workspace_bytes = ws;
    g_launch.clear();
    st = kind == FA_KIND_KVCACHE ? fa_mha_fwd_kvcache(&p, nullptr)
         : kind == FA_KIND_DENSE ? fa_mha_fwd(&p, nullptr)
                                 : fa_mha_varlen_fwd(&p, nullptr);
    EXPECT(st == FA_OK, "%s: forward -> %d (%s)", what, st, fa_last_error());
    int covered = 0;
    for (const Launch& l : g_launch) {
        if (!strcmp(l.kind, "fwd") || !strcmp(l.kind, "decode")) {
            EXPECT(l.B >= 1 && l.B <= 2048, "%s: launch over %d sequences", what, l.B);
            if (!p.cu_seqlens_q) {
                const char* q0 = (const char*)p.q;
                const char* qb = (const char*)l.q;
                // q moves to the chunk's first sequence (unless the decode path
                // swapped in the rotated copy in the workspace)
                if (qb >= q0 && qb < q0 + (int64_t)p.batch * p.q_batch_stride * 2)
                    EXPECT(qb == q0 + (int64_t)covered * p.q_batch_stride * 2, "%s: q offset of chunk %d", what, covered);
                EXPECT(l.lse == p.softmax_lse + (int64_t)covered * p.nheads * p.seqlen_q, "%s: lse offset", what);
            }
            if (p.cache_seqlens) EXPECT(l.seqlens == p.cache_seqlens + covered, "%s: seqlens offset", what);
            covered += l.B;
        }
    }
    EXPECT(covered == p.batch || (p.seqlen_q == 0 && kind != FA_KIND_VARLEN), "%s: %d of %d sequences covered", what,
           covered, p.batch);
}

int main() {
    static int32_t seqlens[5000], cu[5001], table[5000 * 4], bidx[5000];
    for (int i = 0; i < 5000; ++i) {
        seqlens[i] = 37 + i % 900;
        bidx[i] = 4999 - i;
        for (int j = 0; j < 4; ++j) table[i * 4 + j] = i * 4 + j;
    }
    for (int i = 0; i <= 5000; ++i) cu[i] = 3 * i;

    // every batch size around the chunk boundary, decode and prefill shapes
    const int batches[] = {1, 2, 2047, 2048, 2049, 4096, 4097, 5000};
    for (int B : batches) {
        fa_fwd_params p = base(B, 1, 32, 8, 128, 1024);
        p.cache_seqlens = seqlens;
        run_and_check("decode", p, FA_KIND_KVCACHE);
        p.k_new = (const void*)0x600000;
        p.v_new = (const void*)0x680000;
        p.knew_head_stride = p.vnew_head_stride = 128;
        p.knew_row_stride = p.vnew_row_stride = 8 * 128;
        p.knew_batch_stride = p.vnew_batch_stride = 8 * 128;
        p.seqlen_new = 1;
        run_and_check("decode+append", p, FA_KIND_KVCACHE);
        p.block_table = table;
        p.block_table_batch_stride = 4;
        p.max_blocks_per_seq = 4;
        p.block_table_rows = B;
        p.page_block_size = 256;
        p.batch_cache = 4 * B;
        run_and_check("paged decode", p, FA_KIND_KVCACHE);
        p.cache_batch_idx = bidx + (5000 - B);
        run_and_check("paged decode + batch_idx", p, FA_KIND_KVCACHE);

        fa_fwd_params d = base(B, 300, 16, 4, 64, 300);
        run_and_check("dense", d, FA_KIND_DENSE);
        d.num_splits = 3;
        run_and_check("dense split", d, FA_KIND_DENSE);
        fa_fwd_params v = base(B, 3, 8, 2, 128, 0);
        v.cu_seqlens_q = cu;
        v.cu_seqlens_k = cu;
        v.total_q = 3 * B;
        run_and_check("varlen", v, FA_KIND_VARLEN);

        fa_bwd_params b;
        memset(&b, 0, sizeof(b));
        b.abi_version = FA_MI355X_ABI_VERSION;
        b.dtype = FA_DTYPE_FP16;
        b.batch = B;
        b.seqlen_q = b.seqlen_k = 64;
        b.nheads = 8;
        b.nheads_k = 2;
        b.headdim = 128;
        const void* base_ptr = (const void*)0x100000;
        b.q = b.k = b.v = b.out = b.dout = base_ptr;
        b.dq = b.dk = b.dv = (void*)0x200000;
        b.q_row_stride = b.out_row_stride = b.dout_row_stride = b.dq_row_stride = 8 * 128;
        b.k_row_stride = b.v_row_stride = b.dk_row_stride = b.dv_row_stride = 2 * 128;
        b.q_head_stride = b.k_head_stride = b.v_head_stride = b.out_head_stride = b.dout_head_stride = 128;
        b.dq_head_stride = b.dk_head_stride = b.dv_head_stride = 128;
        b.softmax_lse = (const float*)0x300000;
        b.softmax_d = (float*)0x380000;
        b.window_size_left = b.window_size_right = -1;
        g_launch.clear();
        fa_status_t st = fa_mha_bwd(&b, nullptr);
        EXPECT(st == FA_OK, "bwd B=%d -> %d (%s)", B, st, fa_last_error());
        int cov = 0;
        for (const Launch& l : g_launch) {
            EXPECT(l.B <= 2048, "bwd chunk of %d", l.B);
            cov += l.B;
        }
        EXPECT(cov == B, "bwd covered %d of %d", cov, B);
    }

    // invalid and extreme inputs must be refused (or accepted) without UB
    const int32_t weird[] = {0, -1, 1, 7, 8, 256, 257, 65536, 1 << 30, -(1 << 30), 2147483647};
    int refused = 0, accepted = 0;
    for (int32_t x : weird) {
        for (int field = 0; field < 9; ++field) {
            fa_fwd_params p = base(3, 5, 8, 2, 128, 512);
            p.cache_seqlens = seqlens;
            switch (field) {
                case 0: p.batch = x; break;
                case 1: p.seqlen_q = x; break;
                case 2: p.nheads = x; break;
                case 3: p.nheads_k = x; break;
                case 4: p.headdim = p.headdim_v = x; break;
                case 5: p.seqlen_k = x; break;
                case 6: p.num_splits = x; break;
                case 7: p.window_size_left = x; break;
                case 8: p.attention_chunk = x; break;
            }
            for (int kind = 0; kind < 3; ++kind) {
                size_t ws = 0;
                fa_status_t st = fa_fwd_workspace_size(&p, kind, &ws);
                if (st == FA_OK) ++accepted; else ++refused;
                fa_status_t sv = fa_validate(&p, kind);
                EXPECT((st == FA_OK) == (sv == FA_OK), "validate and workspace_size disagree");
            }
        }
    }
    for (int32_t x : weird) {
        for (int field = 0; field < 6; ++field) {
            fa_bwd_params b;
            memset(&b, 0, sizeof(b));
            b.abi_version = FA_MI355X_ABI_VERSION;
            b.dtype = FA_DTYPE_BF16;
            b.batch = 2;
            b.seqlen_q = b.seqlen_k = 40;
            b.nheads = 8;
            b.nheads_k = 2;
            b.headdim = 64;
            b.q = b.k = b.v = b.out = b.dout = (const void*)0x100000;
            b.dq = b.dk = b.dv = (void*)0x200000;
            b.q_row_stride = b.out_row_stride = b.dout_row_stride = b.dq_row_stride = 8 * 64;
            b.k_row_stride = b.v_row_stride = b.dk_row_stride = b.dv_row_stride = 2 * 64;
            b.softmax_lse = (const float*)0x300000;
            b.softmax_d = (float*)0x380000;
            b.window_size_left = b.window_size_right = -1;
            switch (field) {
                case 0: b.batch = x; break;
                case 1: b.seqlen_q = x; break;
                case 2: b.seqlen_k = x; break;
                case 3: b.nheads = x; break;
                case 4: b.nheads_k = x; break;
                case 5: b.headdim = x; break;
            }
            if (fa_validate_bwd(&b, FA_KIND_DENSE) == FA_OK) {
                ++accepted;
                g_launch.clear();
                EXPECT(fa_mha_bwd(&b, nullptr) == FA_OK, "bwd accepted by validation but failed: %s", fa_last_error());
            } else {
                ++refused;
            }
        }
    }
    EXPECT(fa_validate(nullptr, 0) == FA_EINVAL, "null params accepted");
    EXPECT(fa_validate_bwd(nullptr, 1) == FA_EINVAL, "null bwd params accepted");
    printf("harness: %d accepted, %d refused, %d failures\n", accepted, refused, g_fail);
    return g_fail == 0 ? 0 : 1;
}
