// fa_lds_probe.hip -- LDS read-rate probe for gfx950 (MI355X), a measurement
// aid behind the LDS tile layouts of the attention kernels (not part of the
// attention library). One workgroup per CU; each of its waves issues 8
// independent LDS reads per loop iteration to the addresses one access
// pattern of the kernels produces, and the bytes per shader clock per CU come
// from the slowest wave's s_memtime loop time. bench.py --ceilings runs it.
//
// Patterns (16 rows of 256 bytes = a head-dim-128 tile; lane li of lane group
// G reads row li of a 16-row block, chunk 4G + s):
//   0  ds_read_b128, chunk (4G + s) ^ row: the 16-byte operand row read
//   1  ds_read_b64_tr_b16 with swz_v: the V^T transpose read
//   2  ds_read_b64 at the addresses of pattern 1
//   3  two ds_read_b64 per 16-byte operand, halves in the two 128-byte planes
//      of the row, plane h ^ (G & 1) (the split_addr128 scheme)
//   4  two ds_read_b64 per operand, both halves in their natural place
//   5  pattern 3 merged into ds_read2st64_b64 (operands 16 rows apart)
//   6  ds_read2_b64 of a lane's two halves, 128 bytes apart (8 operands)
#include <hip/hip_runtime.h>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef const __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef const __attribute__((address_space(3))) u32x2 lds_u32x2;

constexpr int kReads = 8;

// byte offset of read u of this lane in pattern P (rows of 256 bytes)
template <int P>
__device__ int probe_offset(int wave, int lane, int u) {
    const int li = lane & 15, G = lane >> 4, r4 = li >> 2, c4 = li & 3;
    if constexpr (P == 0) {
        const int row = (u * 16 + wave * 32) % 240 + li;
        return row * 256 + (((G * 4 + (u & 3)) ^ (row & 15)) << 4);
    } else if constexpr (P == 1 || P == 2) {
        const int r = (wave * 16 + u * 16) % 224 + 4 * G + r4;
        const int c = 2 * (u & 7) + (c4 >> 1);
        const int sw = c ^ ((r & 3) << 1) ^ (((r >> 2) & 1) << 3);
        return r * 256 + (sw << 4) + (c4 & 1) * 8;
    } else if constexpr (P == 3 || P == 4) {
        const int row = (u / 2 * 16 + wave * 32) % 240 + li;
        const int c = G * 4 + ((u / 2) & 3);
        const int h = u & 1;
        const int plane = P == 3 ? (h ^ ((c >> 2) & 1)) : 0;
        return row * 256 + plane * 128 + ((c ^ row) & 15) * 8 + (P == 4 ? h * 128 : 0);
    } else if constexpr (P == 5) {
        const int row = (wave * 32) % 192 + li;
        const int c = G * 4;
        return row * 256 + (((u & 1) ^ ((c >> 2) & 1)) * 128) + ((c ^ row) & 15) * 8;
    } else {
        const int row = (u * 16 + wave * 32) % 240 + li;
        const int c = G * 4 + (u & 3);
        return row * 256 + ((c ^ row) & 15) * 8;
    }
}

template <int P>
__global__ void __launch_bounds__(1024, 1) lds_probe_kernel(unsigned* sink, long long* cycles, int iters) {
    __shared__ __attribute__((aligned(256))) unsigned short lds[32768];  // 64 KB
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < 32768; i += blockDim.x) lds[i] = (unsigned short)i;
    __syncthreads();
    int off[kReads];
#pragma unroll
    for (int u = 0; u < kReads; ++u) off[u] = probe_offset<P>(wave, lane, u);
    const char* base = reinterpret_cast<const char*>(lds);
    // every byte read is folded into acc, so each read keeps its own registers
    u32x4 acc[kReads];
#pragma unroll
    for (int u = 0; u < kReads; ++u) acc[u] = u32x4{0u, 0u, 0u, 0u};
    const long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
        // the offsets are opaque each iteration, so no read is hoisted out of the loop
        asm volatile("" : "+v"(off[0]), "+v"(off[1]), "+v"(off[2]), "+v"(off[3]), "+v"(off[4]), "+v"(off[5]),
                     "+v"(off[6]), "+v"(off[7]));
        // every dword read is folded into acc (3-input XORs: one VALU op per
        // two dwords), so each read keeps its own registers and is not narrowed
        unsigned d[kReads * 4];
        constexpr int ND = (P == 0 || P == 6) ? kReads * 4 : kReads * 2;
        if constexpr (P == 0) {
#pragma unroll
            for (int u = 0; u < kReads; ++u) {
                const u32x4 w = *(lds_u32x4*)(base + off[u]);
                d[4 * u] = w[0]; d[4 * u + 1] = w[1]; d[4 * u + 2] = w[2]; d[4 * u + 3] = w[3];
            }
        } else if constexpr (P == 1) {
#pragma unroll
            for (int u = 0; u < kReads; ++u) {
                const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + off[u])));
                d[2 * u] = w[0]; d[2 * u + 1] = w[1];
            }
        } else if constexpr (P >= 2 && P <= 4) {
#pragma unroll
            for (int u = 0; u < kReads; ++u) {
                const u32x2 w = *(lds_u32x2*)(base + off[u]);
                d[2 * u] = w[0]; d[2 * u + 1] = w[1];
            }
        } else if constexpr (P == 5) {
            // one base per half, operands 16 rows (4096 bytes) apart: merged into ds_read2st64_b64
#pragma unroll
            for (int u = 0; u < kReads; ++u) {
                const u32x2 w = *(lds_u32x2*)(base + off[u & 1] + (u >> 1) * 4096);
                d[2 * u] = w[0]; d[2 * u + 1] = w[1];
            }
        } else {
            // a lane's two halves 128 bytes apart: merged into ds_read2_b64
#pragma unroll
            for (int u = 0; u < kReads; ++u) {
                const u32x2 w0 = *(lds_u32x2*)(base + off[u]);
                const u32x2 w1 = *(lds_u32x2*)(base + off[u] + 128);
                d[4 * u] = w0[0]; d[4 * u + 1] = w0[1]; d[4 * u + 2] = w1[0]; d[4 * u + 3] = w1[1];
            }
        }
#pragma unroll
        for (int k = 0; k < ND / 2; ++k) {
            const int u = k % kReads, e = k / kReads % 4;
            acc[u][e] = __builtin_amdgcn_bitop3_b32(acc[u][e], d[2 * k], d[2 * k + 1], 0x96);  // a ^ x ^ y
        }
        __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);  // the reads first, then the XORs
        __builtin_amdgcn_sched_group_barrier(0x002, 64, 0);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const long long t1 = __builtin_amdgcn_s_memtime();
    unsigned x = 0;
#pragma unroll
    for (int u = 0; u < kReads; ++u) x ^= acc[u][0] ^ acc[u][1] ^ acc[u][2] ^ acc[u][3];
    if (x == 0x9e3779b9u) sink[0] = x;  // keeps the reads live
    if (lane == 0) cycles[blockIdx.x * 16 + wave] = t1 - t0;
}

// bytes one wave reads per loop iteration in pattern P
int bytes_per_iter(int p) {
    switch (p) {
        case 0: return kReads * 64 * 16;
        case 1: case 2: case 3: case 4: return kReads * 64 * 8;
        case 5: return kReads * 64 * 8;
        default: return kReads * 64 * 16;
    }
}

}  // namespace

// Runs pattern `pattern` (0..6) with `waves` (1..16) waves per CU on every CU
// of the current device; *bytes_per_clk gets the LDS read rate per CU. Returns
// a hipError_t.
extern "C" int fa_lds_probe(int pattern, int waves, double* bytes_per_clk) {
    if (pattern < 0 || pattern > 6 || waves < 1 || waves > 16 || !bytes_per_clk) return (int)hipErrorInvalidValue;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    int cus = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return (int)e;
    unsigned* sink = nullptr;
    long long* cyc = nullptr;
    if ((e = hipMalloc(&sink, 64)) != hipSuccess) return (int)e;
    if ((e = hipMalloc(&cyc, sizeof(long long) * cus * 16)) != hipSuccess) {
        (void)hipFree(sink);
        return (int)e;
    }
    const int iters = 4096;
    auto launch = [&]() {
        const dim3 g(cus), b(waves * 64);
        switch (pattern) {
            case 0: hipLaunchKernelGGL(lds_probe_kernel<0>, g, b, 0, 0, sink, cyc, iters); break;
            case 1: hipLaunchKernelGGL(lds_probe_kernel<1>, g, b, 0, 0, sink, cyc, iters); break;
            case 2: hipLaunchKernelGGL(lds_probe_kernel<2>, g, b, 0, 0, sink, cyc, iters); break;
            case 3: hipLaunchKernelGGL(lds_probe_kernel<3>, g, b, 0, 0, sink, cyc, iters); break;
            case 4: hipLaunchKernelGGL(lds_probe_kernel<4>, g, b, 0, 0, sink, cyc, iters); break;
            case 5: hipLaunchKernelGGL(lds_probe_kernel<5>, g, b, 0, 0, sink, cyc, iters); break;
            default: hipLaunchKernelGGL(lds_probe_kernel<6>, g, b, 0, 0, sink, cyc, iters); break;
        }
    };
    for (int rep = 0; rep < 2 && e == hipSuccess; ++rep) {  // the first run warms the clocks
        launch();
        e = hipGetLastError();
        if (e == hipSuccess) e = hipDeviceSynchronize();
    }
    long long worst = 0;
    if (e == hipSuccess) {
        long long* h = new long long[(size_t)cus * 16];
        e = hipMemcpy(h, cyc, sizeof(long long) * cus * 16, hipMemcpyDeviceToHost);
        for (int c = 0; c < cus && e == hipSuccess; ++c)
            for (int w = 0; w < waves; ++w) worst = h[c * 16 + w] > worst ? h[c * 16 + w] : worst;
        delete[] h;
    }
    (void)hipFree(sink);
    (void)hipFree(cyc);
    if (e != hipSuccess) return (int)e;
    *bytes_per_clk = worst > 0 ? (double)iters * bytes_per_iter(pattern) * waves / (double)worst : 0.0;
    return 0;
}
