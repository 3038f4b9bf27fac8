/* fa_oracle.h -- CPU checker for the FlashAttention forward path.
 * TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py. The product never links it. */
#ifndef FA_ORACLE_H
#define FA_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_FP16 = 0, ORC_BF16 = 1 };

/* Element strides throughout (not bytes). Head dim is contiguous. */
typedef struct {
    int dtype;
    int B, Sq, Sk, H, Hk, D, Dv;
    const uint16_t* q; int64_t q_sb, q_si, q_sh;
    const int32_t* cu_seqlens_q;           /* varlen q: rows cu[b]..cu[b+1] */
    const uint16_t* k; int64_t k_sb, k_si, k_sh;
    const uint16_t* v; int64_t v_sb, v_si, v_sh;
    const int32_t* seqlens_k;              /* per-batch key count (kvcache) */
    const int32_t* cu_seqlens_k;           /* varlen k */
    const int32_t* block_table; int64_t bt_stride; int page;
    const int32_t* batch_idx;              /* cache_batch_idx */
    const float* alibi; int64_t alibi_sb;  /* slopes[b*alibi_sb + h] */
    float scale, softcap;
    int wl, wr;                            /* normalised window, -1 = unbounded */
    uint16_t* out; int64_t o_sb, o_si, o_sh;
    float* lse; int64_t lse_sb, lse_sh;    /* (B,H,Sq) or, when varlen, (H,T) */
    int nthreads;
    int chunk;                             /* attention_chunk, 0 = off */
    const uint16_t* qv; int64_t qv_sb, qv_si, qv_sh;  /* NULL, or the v3 qv (rows like q, Dv columns):
                                                        the score adds qv . v */
} orc_fwd_params;

typedef struct {
    int dtype, B, S, H, D, rotary_dim, interleaved, q_same_pos;
    uint16_t* x; int64_t x_sb, x_si, x_sh;
    const int32_t* seqlens;
    const uint16_t* cos; const uint16_t* sin; int64_t cs_stride;
} orc_rotary_params;

typedef struct {
    int dtype, B, S_new, Hk, D, Dv, rotary_dim, interleaved;
    const uint16_t* k_new; const uint16_t* v_new; int64_t n_sb, n_si, n_sh;
    uint16_t* k_cache; uint16_t* v_cache; int64_t c_sb, c_si, c_sh;
    const int32_t* seqlens; const int32_t* batch_idx;
    const int32_t* block_table; int64_t bt_stride; int page;
    const uint16_t* cos; const uint16_t* sin; int64_t cs_stride;
    const int32_t* rot_pos;                /* rotary position of token 0 per batch; NULL = seqlens */
} orc_append_params;

float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void orc_normalize_window(int seqlen_q, int seqlen_k, int causal, int* wl, int* wr);
int orc_attention(const orc_fwd_params* p);
int orc_rotary_q(const orc_rotary_params* p);
int orc_kv_append(const orc_append_params* p);
int orc_combine(int S, int64_t R, int Dv, const float* o_part, const float* lse_part, float* o, float* lse);

#ifdef __cplusplus
}
#endif
#endif
