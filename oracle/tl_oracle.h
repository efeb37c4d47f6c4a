/*
 * tl_oracle.h -- CPU oracle for the shared INT8 TinyLlama decoder hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * algorithm (model/tinyllama_gemm_int8.py, model/tinyllama.py and the integer
 * contracts of model/export_fpga_vectors.py and rtl/compute/ SystemVerilog leaves).  It is the
 * reference the HIP path is compared against in the tests, and the timed CPU baseline.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it;
 * the product library never links or calls it.
 *
 * Every function cites the reference file:line it restates.  Pinning status of
 * each function (what checks it against the reference) is listed in the header
 * comment of tl_oracle.c.
 */
#ifndef TL_ORACLE_H
#define TL_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Model geometry; same field order as tl_config in include/tl_int8.h. */
typedef struct or_config {
    int32_t hidden;        /* D   (2048) */
    int32_t intermediate;  /* F   (5632) */
    int32_t n_layers;      /* L   (22)   */
    int32_t n_heads;       /* Hq  (32)   */
    int32_t n_kv_heads;    /* Hkv (4)    */
    int32_t head_dim;      /* hd  (64)   */
    int32_t vocab;         /* V   (32000)*/
    int32_t max_pos;       /* 2048       */
    float   rms_eps;       /* 1e-5       */
    float   rope_theta;    /* 10000      */
} or_config;

/* Weight tensor order inside a layer (model/tinyllama.py:249-267 key order). */
enum { OR_Q = 0, OR_K, OR_V, OR_O, OR_GATE, OR_UP, OR_DOWN, OR_NW };

typedef struct or_layer {
    const int8_t *w[OR_NW];   /* [N][K] int8, output channels K-contiguous */
    const float  *s[OR_NW];   /* [N] fp32 per-output-channel weight scales */
    const float  *g_in;       /* [D] input RMSNorm gain  */
    const float  *g_post;     /* [D] post-attention RMSNorm gain */
} or_layer;

typedef struct or_model {
    or_config       cfg;
    const or_layer *layers;   /* [L] */
    const int8_t   *lm_w;     /* [V][D] */
    const float    *lm_s;     /* [V] */
    const float    *g_final;  /* [D] */
    const int8_t   *emb;      /* [V][D] int8 embedding rows */
    const float    *emb_s;    /* [V] per-row embedding scales */
    const float    *rope_cos; /* [max_pos][hd] */
    const float    *rope_sin; /* [max_pos][hd] */
    const float    *kv_sk;    /* [L][Hkv] static K-cache scales */
    const float    *kv_sv;    /* [L][Hkv] static V-cache scales */
} or_model;

/* Optional per-row capture of intermediate tensors (NULL members skipped). */
typedef struct or_trace {
    float   *attn_in;    /* [D]   RMSNorm output feeding Q/K/V */
    int8_t  *attn_in_q;  /* [D]   */
    double  *attn_in_s;  /* [1]   */
    int32_t *qkv_acc;    /* [D + 2*Hkv*hd] */
    float   *qkv;        /* [D + 2*Hkv*hd] dequantized, before RoPE */
    float   *q_rot;      /* [D]   */
    float   *k_rot;      /* [Hkv*hd] */
    int8_t  *q8;         /* [D]   */
    double  *q_s;        /* [1]   */
    int32_t *scores;     /* [Hq][pos+1] */
    int8_t  *probs;      /* [Hq][pos+1] */
    int32_t *pv_acc;     /* [D]   */
    float   *attended;   /* [D]   */
    float   *x_after_attn; /* [D] */
    float   *hidden;     /* [F]   SiLU(gate)*up */
    float   *out;        /* [D]   layer output */
} or_trace;

/* ---- primitives ---------------------------------------------------------- */
float   or_pairwise_sum(const float *a, int64_t n);
void    or_rms_norm(const float *x, const float *w, int32_t n, float eps, float *out);
double  or_quantize_int8(const float *x, int64_t n, int8_t *q);
void    or_quantize_rows(const float *x, int32_t rows, int32_t cols, int8_t *q, double *scales);
void    or_quantize_weight_rows(const float *w, int32_t rows, int32_t cols, int8_t *q, float *scales);
void    or_quantize_static(const float *x, int64_t n, float scale, int8_t *q);
float   or_dequant_mult(double input_scale, double weight_scale);
void    or_gemm_i8(const int8_t *a, const int8_t *w, int32_t m, int32_t n, int32_t k, int32_t *c);
void    or_requant_f32(const int32_t *acc, const float *mult, int32_t n, int8_t *y);
int8_t  or_requant_q16(int32_t acc, uint32_t mult_q16, int32_t nonnegative_only);
int8_t  or_rotate_q16(int8_t curr, int8_t pair, int32_t cos_q16, int32_t sin_q16, int32_t lower_half);
float   or_expf(float x);
float   or_silu(float x);
float   or_block_sum64(const float *v);
void    or_softmax_row(const float *s, int32_t n, float *p);
void    or_quantize_probs(const float *p, int32_t n, int8_t *p8);
void    or_apply_rope(float *v, int32_t n_heads, int32_t hd, const float *cos_p, const float *sin_p);
int32_t or_argmax_first(const float *v, int32_t n);
int32_t or_argmax_i32_tiles(const int32_t *v, int32_t n, int32_t tile, int32_t *best_val);
void    or_causal_mask_tile(const int32_t *s, int32_t rows, int32_t cols, int32_t qb, int32_t kb, int32_t qrc,
                            int32_t kcc, int32_t *out);

/* ---- attention over the INT8 KV cache ------------------------------------ */
/* K/V cache of one sequence, logical layout [L][Hkv][max_pos][hd] int8. */
void or_attention_row(const or_config *cfg, int32_t layer, int32_t pos,
                      const int8_t *q8, double q_scale,
                      const int8_t *k_cache, const int8_t *v_cache,
                      const float *kv_sk, const float *kv_sv,
                      float *attended, int32_t *scores, int8_t *probs, int32_t *pv_acc);

/* ---- composed path -------------------------------------------------------- */
void    or_embed(const or_model *m, int32_t token, float *x);
void    or_decode_row(const or_model *m, int32_t layer, int32_t pos, float *x,
                      int8_t *k_cache, int8_t *v_cache, or_trace *tr);
int32_t or_lm_head_argmax(const or_model *m, const float *x, float *logits_out, float *best_logit);
/* layer-major multi-row forms of or_decode_row / or_lm_head_argmax (same
 * per-row arithmetic; row r at position pos[r] of the sequence whose caches
 * are k_caches[r] / v_caches[r]) */
void    or_decode_rows(const or_model *m, int32_t layer, int32_t rows, const int32_t *pos, float *x,
                       int8_t *const *k_caches, int8_t *const *v_caches);
void    or_lm_head_rows(const or_model *m, int32_t rows, const float *x, int32_t *tokens, float *best_logits);
int32_t or_forward_token(const or_model *m, int32_t token, int32_t pos, int32_t n_layers,
                         int8_t *k_cache, int8_t *v_cache, float *best_logit);
int32_t or_generate(const or_model *m, const int32_t *prompt, int32_t n_prompt, int32_t max_new,
                    int32_t n_layers, int32_t eos_id, int8_t *k_cache, int8_t *v_cache,
                    int32_t *out_tokens, float *out_logits);

void    or_set_threads(int32_t n);
int32_t or_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
