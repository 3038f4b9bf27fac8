/*
 * fa_oracle.c -- CPU restatement of the reference's FlashAttention forward golden.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product path (the HIP library, the
 * torch extension, the flash_attn_npu_v2/v3 packages) links, loads or calls this
 * file. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * it, as the checker.
 *
 * What it restates (all paths relative to the reference repository root):
 *   - orc_attention: `ref_flash_attention` from tests/test_flash_attn_npu_v3.py:87-146
 *     (identical copy in tests/test_flash_attn_npu_v2.py:84-143):
 *       * keys processed in stacks of 512 (`context_size`, :105);
 *       * S = Q.K^T accumulated in fp32 (`qkMM1`, :49-66), scaled in fp32 (:118);
 *       * softcap c*tanh(s/c) (:121-122);
 *       * masked keys excluded (the golden adds mask*(-1e4), :119,:125; on
 *         rows with at least one visible key the excluded terms are exactly
 *         zero after the online rescale, see orc_attention below);
 *       * online softmax in fp32 (`softmax1`, :29-47), row sum of the fp32 P,
 *         P rounded to the input dtype before P.V (:130), go/gl at the end and
 *         LSE = ln(gl) + gm (:143-146);
 *       * GQA: q head h reads kv head h / (H/Hk) (`group_matmul`, :13-27);
 *       * rows with no visible key: out = 0, lse = +inf (:491-510).
 *   - Mask rule: bottom-right causal / sliding window as in
 *     tests/fa_small_op_golden.py:21-58 and tests/test_flash_attn_npu_v3.py:408-441:
 *     key j is visible to query i iff  j >= i + Sk - Sq - wl (when wl >= 0)
 *     and j <= i + Sk - Sq + wr (when wr >= 0); causal forces wr = 0.
 *   - ALiBi, rotary, in-place append and cache_batch_idx follow the API docstring
 *     in flash_attn_npu_v2/interface_arch22.py:1452-1538 (the reference kernels
 *     reject or ignore them, so the docstring is the only specification):
 *       * alibi: score += -slope[b][h] * |i + Sk - Sq - j| on the scaled score;
 *       * rotary: rotary_dim = 2*cos.shape[1]; interleaved pairs (2i, 2i+1),
 *         GPT-NeoX pairs (i, i + rd/2); fp32 x1*c - x2*s and x2*c + x1*s with
 *         every product rounded to fp32 (no fused multiply-add), then RNE;
 *       * append: cache[idx(b), L_b + t] = rotary(k[b, t]) for t < S_new.
 *   - Paged gather: token j of batch b lives at block block_table[row][j / page],
 *     slot j % page (tests/test_flash_attn_npu_v3.py:444-460).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "fa_oracle.h"

/* ---- 16-bit float conversions (round to nearest even) ---------------------- */

float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t u;
    if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400));
            man &= 0x3ff;
            u = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1f) {
        u = sign | 0x7f800000u | (man << 13);
    } else {
        u = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return sign | (a > 0x7f800000u ? 0x7e00 : 0x7c00);
    if (a >= 0x477ff000u) return sign | 0x7c00; /* rounds to >= 65520 -> inf */
    if (a < 0x38800000u) {                      /* result is subnormal or zero */
        if (a < 0x33000000u) return sign;       /* < 2^-25: rounds to 0 */
        /* value = man * 2^(e-150); the fp16 subnormal unit is 2^-24, so the
         * quotient is man >> (126 - e) with round-to-nearest-even on the rest. */
        uint32_t e = a >> 23;
        uint32_t man = (a & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e;
        uint32_t q = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return sign | (uint16_t)q;
    }
    uint32_t e = (a >> 23) - 127 + 15;
    uint32_t man = a & 0x7fffffu;
    uint32_t q = (e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (q & 1))) q++;
    return sign | (uint16_t)q;
}

static inline float to_f32(int dtype, uint16_t h) {
    return dtype == ORC_BF16 ? orc_bf16_to_f32(h) : orc_f16_to_f32(h);
}

/* The same conversion through a table for fp16 (every one of the 65536 values
 * decoded once by orc_f16_to_f32), for the inner loops of the attention. The
 * table is filled by orc_attention before its parallel region. */
static float g_f16_lut[65536];
static int g_f16_lut_ready = 0;
static void fill_f16_lut(void) {
    if (g_f16_lut_ready) return;
    for (uint32_t h = 0; h < 65536u; h++) g_f16_lut[h] = orc_f16_to_f32((uint16_t)h);
    g_f16_lut_ready = 1;
}
static inline float cvt(int dtype, uint16_t h) {
    if (dtype == ORC_BF16) {
        uint32_t u = (uint32_t)h << 16;
        float f;
        memcpy(&f, &u, 4);
        return f;
    }
    return g_f16_lut[h];
}
static inline uint16_t from_f32(int dtype, float f) {
    return dtype == ORC_BF16 ? orc_f32_to_bf16(f) : orc_f32_to_f16(f);
}
static inline float round_dtype(int dtype, float f) { return to_f32(dtype, from_f32(dtype, f)); }

/* ---- mask / window --------------------------------------------------------- */

/* Window normalisation: tests/fa_small_op_golden.py:21-32 and
 * csrc/arch22/flash_attn_npu_v2/flash_api.cpp:483-494. */
void orc_normalize_window(int seqlen_q, int seqlen_k, int causal, int* wl, int* wr) {
    if (*wl >= seqlen_k - 1) *wl = -1;
    if (*wr >= seqlen_q - 1) *wr = -1;
    if (causal) *wr = 0;
}

/* attention_chunk c > 0 (v3 API, README.md:311-401; the reference rejects it):
 * query i also needs j in [c*floor(d/c), c*floor(d/c) + c), d its diagonal key. */
static inline int key_visible(int i, int j, int sq, int sk, int wl, int wr, int chunk) {
    long d = (long)i + sk - sq; /* diagonal key for query i (bottom-right aligned) */
    if (j < 0 || j >= sk) return 0;
    if (wl >= 0 && j < d - wl) return 0;
    if (wr >= 0 && j > d + wr) return 0;
    if (chunk > 0) {
        long c0 = (long)floor((double)d / (double)chunk) * chunk;
        if (j < c0 || j >= c0 + chunk) return 0;
    }
    return 1;
}

/* ---- the blockwise golden (ref_flash_attention) ----------------------------- */

#define ORC_STACK 512
#define ORC_ROWS 16 /* query rows per unit of parallel work */

static const uint16_t* key_row(const orc_fwd_params* p, int b, int j, int hk, int is_v) {
    const uint16_t* base = is_v ? p->v : p->k;
    int64_t sb = is_v ? p->v_sb : p->k_sb, si = is_v ? p->v_si : p->k_si, sh = is_v ? p->v_sh : p->k_sh;
    if (p->block_table) {
        int row = p->batch_idx ? p->batch_idx[b] : b;
        int blk = p->block_table[(int64_t)row * p->bt_stride + j / p->page];
        return base + (int64_t)blk * sb + (int64_t)(j % p->page) * si + (int64_t)hk * sh;
    }
    if (p->cu_seqlens_k) {
        return base + ((int64_t)p->cu_seqlens_k[b] + j) * si + (int64_t)hk * sh;
    }
    int cb = p->batch_idx ? p->batch_idx[b] : b;
    return base + (int64_t)cb * sb + (int64_t)j * si + (int64_t)hk * sh;
}

static void attention_row(const orc_fwd_params* p, int b, int i, int h, int sq, int sk,
                          float* s, float* pr, uint16_t* out_row, float* lse_out) {
    const int D = p->D, Dv = p->Dv, g = p->H / p->Hk, hk = h / g;
    const int dt = p->dtype;
    int64_t qrow = p->cu_seqlens_q ? ((int64_t)p->cu_seqlens_q[b] + i) * p->q_si
                                   : (int64_t)b * p->q_sb + (int64_t)i * p->q_si;
    const uint16_t* q = p->q + qrow + (int64_t)h * p->q_sh;
    float qf[1024];
    for (int d = 0; d < D; d++) qf[d] = to_f32(dt, q[d]);
    /* qv (FlashAttention-3, flash_attn_npu_v3/interface_arch22.py:1018 of the
     * reference): the score of key j adds qv . v_j, summed after q . k_j in
     * the same fp32 accumulator, i.e. the score of the concatenations [q, qv]
     * and [k_j, v_j] */
    float qvf[1024];
    if (p->qv) {
        int64_t vrow = p->cu_seqlens_q ? ((int64_t)p->cu_seqlens_q[b] + i) * p->qv_si
                                       : (int64_t)b * p->qv_sb + (int64_t)i * p->qv_si;
        const uint16_t* qvr = p->qv + vrow + (int64_t)h * p->qv_sh;
        for (int d = 0; d < Dv; d++) qvf[d] = to_f32(dt, qvr[d]);
    }
    float slope = 0.f;
    if (p->alibi) slope = p->alibi[(int64_t)b * p->alibi_sb + h];

    float go[1024];
    float gl = 0.f, gm = -INFINITY;
    int any = 0;
    int started = 0;
    for (int j0 = 0; j0 < sk; j0 += ORC_STACK) {
        int n = sk - j0 < ORC_STACK ? sk - j0 : ORC_STACK;
        int nvis = 0;
        float lm = -INFINITY;
        int vis[ORC_STACK];
        for (int t = 0; t < n; t++) {
            if (!key_visible(i, j0 + t, sq, sk, p->wl, p->wr, p->chunk)) s[t] = -INFINITY;
            else vis[nvis++] = t;
        }
        /* q . k of the visible keys, four keys at a time: every key keeps its
         * own fp32 accumulator summed in head-dim order (then qv . v in the
         * same accumulator), so each score is what a one-key loop gives */
        float acc[ORC_STACK];
        int u = 0;
        for (; u + 4 <= nvis; u += 4) {
            const uint16_t* k0 = key_row(p, b, j0 + vis[u], hk, 0);
            const uint16_t* k1 = key_row(p, b, j0 + vis[u + 1], hk, 0);
            const uint16_t* k2 = key_row(p, b, j0 + vis[u + 2], hk, 0);
            const uint16_t* k3 = key_row(p, b, j0 + vis[u + 3], hk, 0);
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
            for (int d = 0; d < D; d++) {
                const float qd = qf[d];
                a0 += qd * cvt(dt, k0[d]);
                a1 += qd * cvt(dt, k1[d]);
                a2 += qd * cvt(dt, k2[d]);
                a3 += qd * cvt(dt, k3[d]);
            }
            if (p->qv) {
                const uint16_t* v0 = key_row(p, b, j0 + vis[u], hk, 1);
                const uint16_t* v1 = key_row(p, b, j0 + vis[u + 1], hk, 1);
                const uint16_t* v2 = key_row(p, b, j0 + vis[u + 2], hk, 1);
                const uint16_t* v3 = key_row(p, b, j0 + vis[u + 3], hk, 1);
                for (int d = 0; d < Dv; d++) {
                    const float qd = qvf[d];
                    a0 += qd * cvt(dt, v0[d]);
                    a1 += qd * cvt(dt, v1[d]);
                    a2 += qd * cvt(dt, v2[d]);
                    a3 += qd * cvt(dt, v3[d]);
                }
            }
            acc[u] = a0;
            acc[u + 1] = a1;
            acc[u + 2] = a2;
            acc[u + 3] = a3;
        }
        for (; u < nvis; u++) {
            const uint16_t* kr = key_row(p, b, j0 + vis[u], hk, 0);
            float a = 0.f;
            for (int d = 0; d < D; d++) a += qf[d] * cvt(dt, kr[d]);
            if (p->qv) {
                const uint16_t* vr = key_row(p, b, j0 + vis[u], hk, 1);
                for (int d = 0; d < Dv; d++) a += qvf[d] * cvt(dt, vr[d]);
            }
            acc[u] = a;
        }
        for (u = 0; u < nvis; u++) {
            const int t = vis[u], j = j0 + t;
            float x = acc[u] * p->scale;
            if (p->softcap > 0.f) x = p->softcap * tanhf(x / p->softcap);
            if (p->alibi) {
                long dist = (long)i + sk - sq - j;
                if (dist < 0) dist = -dist;
                x += -slope * (float)dist;
            }
            s[t] = x;
            if (x > lm) lm = x;
        }
        /* A stack with no visible key adds exactly zero once a later stack
         * rescales it (exp(-1e4 - m) underflows in fp32 in the golden); skipping
         * it is the same result. */
        if (nvis == 0) continue;
        any = 1;
        float hm, dm;
        if (!started) { hm = lm; dm = 0.f; }
        else { hm = gm > lm ? gm : lm; dm = gm - hm; }
        gm = hm;
        float row_sum = 0.f;
        for (int t = 0; t < n; t++) {
            float e = (s[t] == -INFINITY) ? 0.f : expf(s[t] - hm);
            row_sum += e;
            pr[t] = round_dtype(dt, e); /* P cast to the input dtype before P.V */
        }
        float lo[1024];
        for (int d = 0; d < Dv; d++) lo[d] = 0.f;
        for (int t = 0; t < n; t++) {
            if (pr[t] == 0.f) continue;
            const uint16_t* vr = key_row(p, b, j0 + t, hk, 1);
            const float pt = pr[t];
            for (int d = 0; d < Dv; d++) lo[d] += pt * cvt(dt, vr[d]);
        }
        if (!started) {
            gl = row_sum;
            for (int d = 0; d < Dv; d++) go[d] = lo[d];
            started = 1;
        } else {
            float e = expf(dm);
            gl = gl * e + row_sum;
            for (int d = 0; d < Dv; d++) go[d] = go[d] * e + lo[d];
        }
    }
    if (!any) {
        for (int d = 0; d < Dv; d++) out_row[d] = from_f32(dt, 0.f);
        *lse_out = INFINITY;
        return;
    }
    for (int d = 0; d < Dv; d++) out_row[d] = from_f32(dt, go[d] / gl);
    *lse_out = logf(gl) + gm;
}

int orc_attention(const orc_fwd_params* p) {
    if (p->D > 1024 || p->Dv > 1024 || p->H % p->Hk) return -1;
    const int B = p->B, H = p->H;
    int nthreads = p->nthreads > 0 ? p->nthreads : 1;
    if (p->dtype != ORC_BF16) fill_f16_lut();
    /* rows are independent: the work is cut into chunks of ORC_ROWS query rows
     * of one (batch, head), so a few long sequences still use every thread */
    int max_sq = 0;
    for (int b = 0; b < B; b++) {
        int sq = p->cu_seqlens_q ? p->cu_seqlens_q[b + 1] - p->cu_seqlens_q[b] : p->Sq;
        if (sq > max_sq) max_sq = sq;
    }
    const int64_t nchunk = (max_sq + ORC_ROWS - 1) / ORC_ROWS;
    const int64_t nwork = (int64_t)B * H * nchunk;
#pragma omp parallel num_threads(nthreads)
    {
        float* s = (float*)malloc(sizeof(float) * ORC_STACK);
        float* pr = (float*)malloc(sizeof(float) * ORC_STACK);
#pragma omp for schedule(dynamic, 1)
        for (int64_t w = 0; w < nwork; w++) {
            {
                const int b = (int)(w / ((int64_t)H * nchunk));
                const int h = (int)((w / nchunk) % H);
                const int i0 = (int)(w % nchunk) * ORC_ROWS;
                int sq = p->cu_seqlens_q ? p->cu_seqlens_q[b + 1] - p->cu_seqlens_q[b] : p->Sq;
                int sk = p->seqlens_k ? p->seqlens_k[b]
                       : (p->cu_seqlens_k ? p->cu_seqlens_k[b + 1] - p->cu_seqlens_k[b] : p->Sk);
                const int i1 = i0 + ORC_ROWS < sq ? i0 + ORC_ROWS : sq;
                for (int i = i0; i < i1; i++) {
                    int64_t orow = p->cu_seqlens_q ? ((int64_t)p->cu_seqlens_q[b] + i) * p->o_si
                                                   : (int64_t)b * p->o_sb + (int64_t)i * p->o_si;
                    uint16_t* o = p->out + orow + (int64_t)h * p->o_sh;
                    float* l;
                    if (p->cu_seqlens_q) l = p->lse + (int64_t)h * p->lse_sh + p->cu_seqlens_q[b] + i;
                    else l = p->lse + (int64_t)b * p->lse_sb + (int64_t)h * p->lse_sh + i;
                    attention_row(p, b, i, h, sq, sk, s, pr, o, l);
                }
            }
        }
        free(s);
        free(pr);
    }
    return 0;
}

/* ---- rotary + append --------------------------------------------------------- */

/* Rotate one head vector x[0..D) in place at position pos. cos/sin are
 * (seqlen_ro, rd/2) in the storage dtype. Products rounded to fp32 separately
 * (volatile stores keep the compiler from contracting them into an FMA). */
static void rotate_vec(int dt, uint16_t* x, int D, int rd, int interleaved,
                       const uint16_t* cos_row, const uint16_t* sin_row) {
    uint16_t tmp[1024];
    memcpy(tmp, x, sizeof(uint16_t) * D);
    int half = rd / 2;
    for (int i = 0; i < half; i++) {
        int i1 = interleaved ? 2 * i : i;
        int i2 = interleaved ? 2 * i + 1 : i + half;
        float c = to_f32(dt, cos_row[i]), s = to_f32(dt, sin_row[i]);
        float x1 = to_f32(dt, tmp[i1]), x2 = to_f32(dt, tmp[i2]);
        volatile float a = x1 * c, bb = x2 * s, cc = x2 * c, dd = x1 * s;
        float o1 = a - bb;
        float o2 = cc + dd;
        x[i1] = from_f32(dt, o1);
        x[i2] = from_f32(dt, o2);
    }
}

int orc_rotary_q(const orc_rotary_params* p) {
    for (int b = 0; b < p->B; b++) {
        int L = p->seqlens ? p->seqlens[b] : 0;
        for (int i = 0; i < p->S; i++) {
            int pos = L + (p->q_same_pos ? 0 : i);
            const uint16_t* cr = p->cos + (int64_t)pos * p->cs_stride;
            const uint16_t* sr = p->sin + (int64_t)pos * p->cs_stride;
            for (int h = 0; h < p->H; h++) {
                uint16_t* x = p->x + (int64_t)b * p->x_sb + (int64_t)i * p->x_si + (int64_t)h * p->x_sh;
                rotate_vec(p->dtype, x, p->D, p->rotary_dim, p->interleaved, cr, sr);
            }
        }
    }
    return 0;
}

int orc_kv_append(const orc_append_params* p) {
    uint16_t buf[1024];
    for (int b = 0; b < p->B; b++) {
        int L = p->seqlens[b];
        int row = p->batch_idx ? p->batch_idx[b] : b;
        for (int t = 0; t < p->S_new; t++) {
            int j = L + t;
            for (int h = 0; h < p->Hk; h++) {
                for (int which = 0; which < 2; which++) {
                    const uint16_t* src = (which ? p->v_new : p->k_new) + (int64_t)b * p->n_sb +
                                          (int64_t)t * p->n_si + (int64_t)h * p->n_sh;
                    int Dw = which ? p->Dv : p->D;
                    memcpy(buf, src, sizeof(uint16_t) * Dw);
                    if (!which && p->cos) {
                        /* rotary at rotary_seqlens[b] + t when given (v3), else at the slot */
                        const int64_t pos = p->rot_pos ? (int64_t)p->rot_pos[b] + t : j;
                        const uint16_t* cr = p->cos + pos * p->cs_stride;
                        const uint16_t* sr = p->sin + pos * p->cs_stride;
                        rotate_vec(p->dtype, buf, Dw, p->rotary_dim, p->interleaved, cr, sr);
                    }
                    uint16_t* cache = which ? p->v_cache : p->k_cache;
                    uint16_t* dst;
                    if (p->block_table) {
                        int blk = p->block_table[(int64_t)row * p->bt_stride + j / p->page];
                        dst = cache + (int64_t)blk * p->c_sb + (int64_t)(j % p->page) * p->c_si + (int64_t)h * p->c_sh;
                    } else {
                        dst = cache + (int64_t)row * p->c_sb + (int64_t)j * p->c_si + (int64_t)h * p->c_sh;
                    }
                    memcpy(dst, buf, sizeof(uint16_t) * Dw);
                }
            }
        }
    }
    return 0;
}

/* ---- split-KV combine --------------------------------------------------------- */

/* lse = m + ln sum_i exp(lse_i - m); O = sum_i exp(lse_i - lse) * O_i
 * (csrc/arch22/flash_attn_npu_v2/CombineScale.hpp:150-194, :248-316).
 * Partials: o_part[s][r][Dv] fp32, lse_part[s][r]; rows r = 0..R-1. */
int orc_combine(int S, int64_t R, int Dv, const float* o_part, const float* lse_part,
                float* o, float* lse) {
    for (int64_t r = 0; r < R; r++) {
        /* A split that saw no visible key carries a non-finite LSE and adds nothing. */
        float m = -INFINITY;
        for (int s = 0; s < S; s++) {
            float v = lse_part[(int64_t)s * R + r];
            if (isfinite(v) && v > m) m = v;
        }
        if (m == -INFINITY) {
            for (int d = 0; d < Dv; d++) o[r * Dv + d] = 0.f;
            lse[r] = INFINITY;
            continue;
        }
        float sum = 0.f;
        for (int s = 0; s < S; s++) {
            float v = lse_part[(int64_t)s * R + r];
            if (isfinite(v)) sum += expf(v - m);
        }
        float l = m + logf(sum);
        lse[r] = l;
        for (int d = 0; d < Dv; d++) {
            float acc = 0.f;
            for (int s = 0; s < S; s++) {
                float v = lse_part[(int64_t)s * R + r];
                if (!isfinite(v)) continue;
                acc += expf(v - l) * o_part[((int64_t)s * R + r) * Dv + d];
            }
            o[r * Dv + d] = acc;
        }
    }
    return 0;
}
