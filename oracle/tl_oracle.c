/*
 * tl_oracle.c -- CPU oracle (TEST INFRASTRUCTURE, never part of the product).
 *
 * Plain-C restatement of the reference's INT8 decoder path.  The reference is a
 * NumPy golden model (model/tinyllama_gemm_int8.py "GI", model/tinyllama.py
 * "TL") plus integer contracts in model/export_fpga_vectors.py ("EX") and the
 * SystemVerilog leaves under rtl/compute/.  Generalisations the reference's
 * spec asks for (docs/design_decisions.txt A7, A10, B1, B2) and the golden does
 * not implement are stated where they are made:
 *   - weights carry static per-output-channel fp32 scales (A10, B1);
 *   - activations are quantized per row (per token); at one row this is the
 *     golden's per-tensor quantize_int8 (GI:36-42) exactly;
 *   - attention runs over a symmetric INT8 KV cache with static per-layer,
 *     per-KV-head scales (A7, B2), with INT8xINT8->INT32 score and
 *     probability-times-V contractions (A9; EX:870-873, EX:2082-2089).
 *
 * Floating-point operations follow NumPy's evaluation order exactly where the
 * golden fixes it (pairwise summation in np.mean, weak-scalar promotion of
 * Python floats to float32).  Where NumPy's bits come from its own SIMD
 * transcendental code (np.exp) the oracle uses its own exp (or_expf) and the
 * HIP kernels use the same function, so the oracle and the GPU agree bit for
 * bit; the oracle is pinned to the golden within a stated tolerance there.
 *
 * Pinning (tests that tie each function to the reference; see tests/):
 *   or_pairwise_sum, or_rms_norm   bit-exact vs golden rms_norm vectors (TL:45-50)
 *   or_quantize_int8/_rows         bit-exact vs golden quantize_int8 vectors and
 *                                  sim/test_k16, sim/test_k64 fixtures
 *   or_dequant_mult                bit-exact vs golden dequantize_int32 vectors
 *   or_gemm_i8                     sim/{x,w,expected}.txt, sim/test_k*, MAC KATs,
 *                                  brute-force int64 products
 *   or_requant_f32                 equals or_requant_q16 wherever the Q16.16
 *                                  multiplier is exact; requantize_unit KATs
 *   or_requant_q16, or_rotate_q16  tb_requantize_unit / tb_rope_unit KATs and
 *                                  the rope_{cos,sin}_rom.memh tables
 *   or_expf                        against libm exp in double, <= 2 ulp
 *   or_silu, or_softmax_row        golden vectors within 1e-6 relative
 *   or_apply_rope                  bit-exact vs golden apply_rope vectors
 *   or_quantize_probs              bit-exact vs EX:870-873 restated probabilities
 *   or_attention_row               integer parts by brute force; end result vs
 *                                  the golden float attention within the INT8
 *                                  quantization tolerance
 *   or_decode_row                  vs golden mixed_precision_decoder_layer at one
 *                                  token within tolerance
 *   or_lm_head_argmax              argmax_reduction KATs (lower id wins a tie)
 *   or_argmax_i32_tiles            argmax_reduction KATs; np.argmax on random
 *                                  INT32 vectors with forced ties
 *   or_causal_mask_tile            tb_causal_mask_unit KAT (col 0 kept, cols
 *                                  1-4 masked, inactive row 0); brute-force
 *                                  restatement of the allow rule
 *   or_decode_rows, or_lm_head_rows  bit-exact vs or_decode_row / or_lm_head_argmax
 *                                  row by row (prompt rows of one sequence and
 *                                  rows of different sequences)
 */
#include "tl_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void or_set_threads(int32_t n) {
    g_threads = n < 1 ? 1 : n;
#ifdef _OPENMP
    omp_set_num_threads(g_threads);
#endif
}

int32_t or_get_threads(void) { return g_threads; }

/* NumPy pairwise summation of a contiguous float32 run (the reduction np.mean
 * uses for float32 along a contiguous axis; blocks of 128 with eight
 * accumulators, recursive halving on multiples of eight above that). */
float or_pairwise_sum(const float *a, int64_t n) {
    if (n < 8) {
        float res = 0.0f;
        for (int64_t i = 0; i < n; i++) res = res + a[i];
        return res;
    }
    if (n <= 128) {
        float r[8];
        int64_t i;
        for (int j = 0; j < 8; j++) r[j] = a[j];
        for (i = 8; i < n - (n % 8); i += 8)
            for (int j = 0; j < 8; j++) r[j] = r[j] + a[i + j];
        float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        for (; i < n; i++) res = res + a[i];
        return res;
    }
    int64_t n2 = n / 2;
    n2 -= n2 % 8;
    return or_pairwise_sum(a, n2) + or_pairwise_sum(a + n2, n - n2);
}

/* TL:45-50  x * (1/sqrt(mean(x*x) + eps)) * w, all float32. */
void or_rms_norm(const float *x, const float *w, int32_t n, float eps, float *out) {
    float *sq = (float *)malloc(sizeof(float) * (size_t)n);
    for (int32_t i = 0; i < n; i++) sq[i] = x[i] * x[i];
    float var = or_pairwise_sum(sq, n) / (float)n;
    float inv = 1.0f / sqrtf(var + eps);
    for (int32_t i = 0; i < n; i++) out[i] = (x[i] * inv) * w[i];
    free(sq);
}

static inline int8_t sat_i8(float v) {
    if (v > 127.0f) v = 127.0f;
    if (v < -127.0f) v = -127.0f;
    return (int8_t)v;
}

/* GI:36-42  scale = max|x| / 127 in float64 (1.0 when all zero); the divide
 * uses the scale rounded to float32 (NumPy weak-scalar rule); np.round is
 * round-half-to-even; clip to +-127 (never -128). */
double or_quantize_int8(const float *x, int64_t n, int8_t *q) {
    float mx = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        if (a > mx) mx = a;
    }
    double s = (n > 0 && mx != 0.0f) ? (double)mx / 127.0 : 1.0;
    float sf = (float)s;
    for (int64_t i = 0; i < n; i++) q[i] = sat_i8(rintf(x[i] / sf));
    return s;
}

/* Per-row application of GI:36-42 (the per-token activation scale that a KV
 * cache needs; identical to the golden at one row). */
void or_quantize_rows(const float *x, int32_t rows, int32_t cols, int8_t *q, double *scales) {
    for (int32_t r = 0; r < rows; r++)
        scales[r] = or_quantize_int8(x + (int64_t)r * cols, cols, q + (int64_t)r * cols);
}

/* Offline per-output-channel weight quantizer: GI:36-42 applied to each
 * [N][K] row, the scale stored as float32 (design_decisions A10 / B1). */
void or_quantize_weight_rows(const float *w, int32_t rows, int32_t cols, int8_t *q, float *scales) {
    for (int32_t r = 0; r < rows; r++)
        scales[r] = (float)or_quantize_int8(w + (int64_t)r * cols, cols, q + (int64_t)r * cols);
}

/* Quantize with a given static scale: GI:40-41 with the scale supplied
 * (KV-cache rows, design_decisions A7/A10). */
void or_quantize_static(const float *x, int64_t n, float scale, int8_t *q) {
    for (int64_t i = 0; i < n; i++) q[i] = sat_i8(rintf(x[i] / scale));
}

/* GI:45-46  the multiplier (input_scale * weight_scale) is formed in float64
 * and rounded once to float32 when it meets the float32 accumulator array. */
float or_dequant_mult(double input_scale, double weight_scale) {
    return (float)(input_scale * weight_scale);
}

/* GI:70 / shared_gemm_engine.sv:126-135  C[m][n] = sum_k A[m][k] * W[n][k]
 * with int32 accumulation (|acc| <= K * 127^2 < 2^31 for K <= 133,000). */
void or_gemm_i8(const int8_t *a, const int8_t *w, int32_t m, int32_t n, int32_t k, int32_t *c) {
#pragma omp parallel for schedule(static)
    for (int32_t j = 0; j < n; j++) {
        const int8_t *wr = w + (int64_t)j * k;
        int32_t i = 0;
        /* four rows per pass over the weight row (exact integer sums, so the
         * grouping changes nothing but speed) */
        for (; i + 4 <= m; i += 4) {
            const int8_t *a0 = a + (int64_t)i * k, *a1 = a0 + k, *a2 = a1 + k, *a3 = a2 + k;
            int32_t s0 = 0, s1 = 0, s2 = 0, s3 = 0;
            for (int32_t t = 0; t < k; t++) {
                const int32_t wv = wr[t];
                s0 += (int32_t)a0[t] * wv;
                s1 += (int32_t)a1[t] * wv;
                s2 += (int32_t)a2[t] * wv;
                s3 += (int32_t)a3[t] * wv;
            }
            c[(int64_t)i * n + j] = s0;
            c[(int64_t)(i + 1) * n + j] = s1;
            c[(int64_t)(i + 2) * n + j] = s2;
            c[(int64_t)(i + 3) * n + j] = s3;
        }
        for (; i < m; i++) {
            const int8_t *ar = a + (int64_t)i * k;
            int32_t s = 0;
            for (int32_t t = 0; t < k; t++) s += (int32_t)ar[t] * (int32_t)wr[t];
            c[(int64_t)i * n + j] = s;
        }
    }
}

/* Requantize INT32 -> INT8 with a float32 multiplier per output channel:
 * y = sat+-127(rne(float(acc) * m)).  The fp32 form of requantize_unit.sv:39-93
 * (whose multiplier is unsigned Q16.16). */
void or_requant_f32(const int32_t *acc, const float *mult, int32_t n, int8_t *y) {
    for (int32_t i = 0; i < n; i++) y[i] = sat_i8(rintf((float)acc[i] * mult[i]));
}

static int64_t rne_shift16(int64_t prod) {
    uint64_t mag = (uint64_t)(prod < 0 ? -prod : prod);
    uint64_t quo = mag >> 16;
    uint64_t rem = mag & 0xFFFFu;
    if (rem > 0x8000u || (rem == 0x8000u && (quo & 1u))) quo += 1;
    return prod < 0 ? -(int64_t)quo : (int64_t)quo;
}

/* requantize_unit.sv:39-93  product with an unsigned Q16.16 multiplier,
 * round half to even on the 16 fraction bits, clamp to +-127 (or [0,127]). */
int8_t or_requant_q16(int32_t acc, uint32_t mult_q16, int32_t nonnegative_only) {
    int64_t r = rne_shift16((int64_t)acc * (int64_t)mult_q16);
    if (nonnegative_only) {
        if (r < 0) r = 0;
        if (r > 127) r = 127;
    } else {
        if (r > 127) r = 127;
        if (r < -127) r = -127;
    }
    return (int8_t)r;
}

/* rope_unit.sv:73-127 / EX:684-697  INT8 RoPE with Q16.16 cos/sin: lower half
 * computes curr*cos - pair*sin, upper half curr*cos + pair*sin, RNE, +-127. */
int8_t or_rotate_q16(int8_t curr, int8_t pair, int32_t cos_q16, int32_t sin_q16, int32_t lower_half) {
    int64_t c = (int64_t)curr * cos_q16;
    int64_t p = (int64_t)pair * sin_q16;
    int64_t r = rne_shift16(lower_half ? c - p : c + p);
    if (r > 127) r = 127;
    if (r < -127) r = -127;
    return (int8_t)r;
}

/* exp(x) in float32 shared bit-for-bit with the HIP kernels.  Cody-Waite
 * reduction x = k*ln2 + r with ln2 split as 355/512 + (ln2 - 355/512), then the
 * degree-7 Taylor polynomial of e^r (coefficients 1/n! rounded to float32) in
 * Horner form with fused multiply-adds, scaled by 2^k built from the exponent
 * field.  Inputs below -80 return 0 (their softmax weight underflows anyway);
 * the callers never pass more than +60. */
float or_expf(float x) {
    if (!(x >= -80.0f)) return 0.0f;
    if (x > 80.0f) x = 80.0f;
    const float log2e = 0x1.715476p+0f;
    const float c1 = 0x1.63p-1f;         /* 355/512 */
    const float c2 = -0x1.bd0106p-13f;   /* ln2 - 355/512 */
    float kf = rintf(x * log2e);
    float r = fmaf(-kf, c1, x);
    r = fmaf(-kf, c2, r);
    float p = 0x1.a01a02p-13f;           /* 1/5040 */
    p = fmaf(p, r, 0x1.6c16c2p-10f);     /* 1/720  */
    p = fmaf(p, r, 0x1.111112p-7f);      /* 1/120  */
    p = fmaf(p, r, 0x1.555556p-5f);      /* 1/24   */
    p = fmaf(p, r, 0x1.555556p-3f);      /* 1/6    */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int32_t k = (int32_t)kf;
    uint32_t bits = (uint32_t)(k + 127) << 23;
    float two_k;
    memcpy(&two_k, &bits, sizeof two_k);
    return p * two_k;
}

/* TL:159-161  x / (1 + exp(-clip(x, -60, 60))) in float32. */
float or_silu(float x) {
    float c = x < -60.0f ? -60.0f : (x > 60.0f ? 60.0f : x);
    return x / (1.0f + or_expf(-c));
}

/* Sum of 64 values by the xor butterfly a wavefront uses: at each level
 * (offsets 32,16,8,4,2,1) every slot i becomes v[i] + v[i ^ off]. */
float or_block_sum64(const float *v) {
    float a[64], b[64];
    memcpy(a, v, sizeof a);
    for (int off = 32; off >= 1; off >>= 1) {
        for (int i = 0; i < 64; i++) b[i] = a[i] + a[i ^ off];
        memcpy(a, b, sizeof a);
    }
    return a[0];
}

/* TL:100-103 softmax(x) = exp(x - max) / sum(exp(x - max)), float32.  The sum
 * runs over blocks of 64 consecutive keys: each block is reduced by the
 * butterfly above (missing keys count as 0), and block sums are added in key
 * order starting from 0. */
void or_softmax_row(const float *s, int32_t n, float *p) {
    if (n <= 0) return;
    float m = s[0];
    for (int32_t t = 1; t < n; t++)
        if (s[t] > m) m = s[t];
    float blk[64];
    float total = 0.0f;
    for (int32_t b = 0; b * 64 < n; b++) {
        for (int j = 0; j < 64; j++) {
            int32_t t = b * 64 + j;
            blk[j] = t < n ? or_expf(s[t] - m) : 0.0f;
            if (t < n) p[t] = blk[j];
        }
        total = total + or_block_sum64(blk);
    }
    for (int32_t t = 0; t < n; t++) p[t] = p[t] / total;
}

/* EX:870-873  probabilities to INT8: rne(p * 127) clipped to [0, 127]
 * (fixed probability scale 1/127, softmax_wrapper.sv:23). */
void or_quantize_probs(const float *p, int32_t n, int8_t *p8) {
    for (int32_t t = 0; t < n; t++) {
        float v = rintf(p[t] * 127.0f);
        if (v < 0.0f) v = 0.0f;
        if (v > 127.0f) v = 127.0f;
        p8[t] = (int8_t)v;
    }
}

/* TL:69-80  q*cos + rotate_half(q)*sin for every head of one token, where
 * rotate_half(q) = concat(-q[hd/2:], q[:hd/2]). */
void or_apply_rope(float *v, int32_t n_heads, int32_t hd, const float *cos_p, const float *sin_p) {
    int32_t half = hd / 2;
    float *tmp = (float *)malloc(sizeof(float) * (size_t)hd);
    for (int32_t h = 0; h < n_heads; h++) {
        float *x = v + (int64_t)h * hd;
        for (int32_t d = 0; d < hd; d++) {
            float rot = d < half ? -x[d + half] : x[d - half];
            tmp[d] = (x[d] * cos_p[d]) + (rot * sin_p[d]);
        }
        memcpy(x, tmp, sizeof(float) * (size_t)hd);
    }
    free(tmp);
}

/* GI:671 np.argmax: index of the first maximum (design_decisions B4: the lower
 * token id wins a tie). */
int32_t or_argmax_first(const float *v, int32_t n) {
    int32_t best = 0;
    for (int32_t i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

/* argmax_reduction.sv:47-93 over INT32 logits delivered in vocab tiles: the
 * per-tile winner and the running winner use (logit greater) or (equal and
 * lower id). */
int32_t or_argmax_i32_tiles(const int32_t *v, int32_t n, int32_t tile, int32_t *best_val) {
    int32_t best_id = 0, best = 0, have = 0;
    for (int32_t base = 0; base < n; base += tile) {
        int32_t cnt = n - base < tile ? n - base : tile;
        int32_t tid = base, tv = v[base];
        for (int32_t j = 1; j < cnt; j++)
            if (v[base + j] > tv) { tv = v[base + j]; tid = base + j; }
        if (!have || tv > best || (tv == best && tid < best_id)) { best = tv; best_id = tid; have = 1; }
    }
    if (best_val) *best_val = best;
    return best_id;
}

/* causal_mask_unit.sv:37-54 / EX:1157-1184  one tile of INT32 scores
 * [rows][cols]: (r, c) keeps its score when r < qrc, c < kcc and
 * kb + c <= qb + r; the rest of an active row is MASK_NEG_INF (-1e9,
 * tinyllama_pkg.sv), rows r >= qrc are 0. */
void or_causal_mask_tile(const int32_t *s, int32_t rows, int32_t cols, int32_t qb, int32_t kb, int32_t qrc,
                         int32_t kcc, int32_t *out) {
    for (int32_t r = 0; r < rows; r++)
        for (int32_t c = 0; c < cols; c++) {
            const int64_t i = (int64_t)r * cols + c;
            if (r >= qrc) out[i] = 0;
            else out[i] = (c < kcc && (int64_t)kb + c <= (int64_t)qb + r) ? s[i] : -1000000000;
        }
}

static inline int64_t cache_row(const or_config *c, int32_t layer, int32_t g, int32_t t) {
    /* kv_cache_manager.sv:43-44 row index ((layer*Hkv + kv_head)*MAX_POS + token) */
    return (((int64_t)layer * c->n_kv_heads + g) * c->max_pos + t) * c->head_dim;
}

/* One query row of GQA attention over the INT8 cache (keys 0..pos):
 *   q head h reads kv head h / (Hq/Hkv)           (gqa_router.sv:29, TL:94-97)
 *   S[t] = sum_d q8[d] * k8[t][d]                 (INT32, EX:1251)
 *   s[t] = float(S[t]) * f32((s_q*s_k)*attn_scale) (EX:2082-2089, GI:158)
 *   p = softmax(s); p8 = rne(127 p) in [0,127]    (TL:100-103, EX:870-873)
 *   O[d] = sum_t p8[t] * v8[t][d]                 (INT32, gemm_operand_router P x V)
 *   attended = float(O) * f32((1/127) * s_v)      (GI:45-46 with the 1/127 scale)
 * Keys after pos are causally masked (causal_mask_unit.sv:49-54) and simply
 * not visited: their -1e9 scores give exp() == 0 in the golden. */
void or_attention_row(const or_config *cfg, int32_t layer, int32_t pos,
                      const int8_t *q8, double q_scale,
                      const int8_t *k_cache, const int8_t *v_cache,
                      const float *kv_sk, const float *kv_sv,
                      float *attended, int32_t *scores, int8_t *probs, int32_t *pv_acc) {
    const int32_t hd = cfg->head_dim, hq = cfg->n_heads, hkv = cfg->n_kv_heads;
    const int32_t groups = hq / hkv, n = pos + 1;
    if (hd > 256) abort();
    const double attn_scale = 1.0 / sqrt((double)hd);
    int32_t *S = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
    float *s = (float *)malloc(sizeof(float) * (size_t)n);
    float *p = (float *)malloc(sizeof(float) * (size_t)n);
    int8_t *p8 = (int8_t *)malloc((size_t)n);
    for (int32_t h = 0; h < hq; h++) {
        const int32_t g = h / groups;
        const int8_t *q = q8 + (int64_t)h * hd;
        const int8_t *kb = k_cache + cache_row(cfg, layer, g, 0);
        const int8_t *vb = v_cache + cache_row(cfg, layer, g, 0);
        const float sk = kv_sk[layer * hkv + g], sv = kv_sv[layer * hkv + g];
        const float sc = (float)((q_scale * (double)sk) * attn_scale);
        for (int32_t t = 0; t < n; t++) {
            int32_t acc = 0;
            for (int32_t d = 0; d < hd; d++) acc += (int32_t)q[d] * (int32_t)kb[(int64_t)t * hd + d];
            S[t] = acc;
            s[t] = (float)acc * sc;
        }
        or_softmax_row(s, n, p);
        or_quantize_probs(p, n, p8);
        const float pv_mult = or_dequant_mult(1.0 / 127.0, (double)sv);
        /* integer sums are exact, so visiting the keys row by row (the cache's
         * contiguous order) gives the same accumulators as any other order */
        int32_t acc[256];
        for (int32_t d = 0; d < hd; d++) acc[d] = 0;
        for (int32_t t = 0; t < n; t++) {
            const int8_t *vr = vb + (int64_t)t * hd;
            const int32_t pt = p8[t];
            if (pt == 0) continue;
            for (int32_t d = 0; d < hd; d++) acc[d] += pt * (int32_t)vr[d];
        }
        for (int32_t d = 0; d < hd; d++) {
            if (pv_acc) pv_acc[h * hd + d] = acc[d];
            attended[h * hd + d] = (float)acc[d] * pv_mult;
        }
        if (scores) memcpy(scores + (int64_t)h * n, S, sizeof(int32_t) * (size_t)n);
        if (probs) memcpy(probs + (int64_t)h * n, p8, (size_t)n);
    }
    free(S); free(s); free(p); free(p8);
}

/* Embedding row of the INT8 table (embedding_quantizer.sv path; the golden's
 * weights.embed TL:240-241 returns the same float32 row). */
void or_embed(const or_model *m, int32_t token, float *x) {
    const int32_t D = m->cfg.hidden;
    const int8_t *row = m->emb + (int64_t)token * D;
    const float s = m->emb_s[token];
    for (int32_t d = 0; d < D; d++) x[d] = (float)row[d] * s;
}

/* Quantized projection of one row: quantize x (GI:68), int32 contraction
 * (GI:70), per-output-channel dequantization (GI:45-46, 71). */
static void linear_row(const int8_t *x8, double sx, const int8_t *w, const float *ws,
                       int32_t n, int32_t k, float *y, int32_t *acc_out) {
    int32_t *acc = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
    or_gemm_i8(x8, w, 1, n, k, acc);
    for (int32_t j = 0; j < n; j++) y[j] = (float)acc[j] * or_dequant_mult(sx, (double)ws[j]);
    if (acc_out) memcpy(acc_out, acc, sizeof(int32_t) * (size_t)n);
    free(acc);
}

/* One decoder layer for one token at position pos (GI:256-281 with the
 * attention of GI:136-182 over the INT8 KV cache), updating x in place and
 * appending this token's K/V rows.  k_cache / v_cache are the sequence's
 * [L][Hkv][max_pos][hd] int8 buffers. */
void or_decode_row(const or_model *m, int32_t layer, int32_t pos, float *x,
                   int8_t *k_cache, int8_t *v_cache, or_trace *tr) {
    const or_config *c = &m->cfg;
    const or_layer *L = &m->layers[layer];
    const int32_t D = c->hidden, F = c->intermediate, hd = c->head_dim;
    const int32_t hkv = c->n_kv_heads, kvd = hkv * hd;
    float *a = (float *)malloc(sizeof(float) * (size_t)D);
    int8_t *a8 = (int8_t *)malloc((size_t)(D > F ? D : F));
    float *qkv = (float *)malloc(sizeof(float) * (size_t)(D + 2 * kvd));
    float *att = (float *)malloc(sizeof(float) * (size_t)D);
    float *o = (float *)malloc(sizeof(float) * (size_t)D);
    float *gt = (float *)malloc(sizeof(float) * (size_t)F);
    float *up = (float *)malloc(sizeof(float) * (size_t)F);
    int8_t *q8 = (int8_t *)malloc((size_t)D);
    int8_t *kv8 = (int8_t *)malloc((size_t)kvd);

    /* GI:264 attention input */
    or_rms_norm(x, L->g_in, D, c->rms_eps, a);
    double sa = or_quantize_int8(a, D, a8);
    if (tr && tr->attn_in) memcpy(tr->attn_in, a, sizeof(float) * (size_t)D);
    if (tr && tr->attn_in_q) memcpy(tr->attn_in_q, a8, (size_t)D);
    if (tr && tr->attn_in_s) tr->attn_in_s[0] = sa;
    /* GI:146-148 Q/K/V projections */
    linear_row(a8, sa, L->w[OR_Q], L->s[OR_Q], D, D, qkv, tr ? tr->qkv_acc : NULL);
    linear_row(a8, sa, L->w[OR_K], L->s[OR_K], kvd, D, qkv + D, tr && tr->qkv_acc ? tr->qkv_acc + D : NULL);
    linear_row(a8, sa, L->w[OR_V], L->s[OR_V], kvd, D, qkv + D + kvd, tr && tr->qkv_acc ? tr->qkv_acc + D + kvd : NULL);
    if (tr && tr->qkv) memcpy(tr->qkv, qkv, sizeof(float) * (size_t)(D + 2 * kvd));
    /* GI:154 RoPE on Q and K at this position */
    const float *cp = m->rope_cos + (int64_t)pos * hd, *sp = m->rope_sin + (int64_t)pos * hd;
    or_apply_rope(qkv, c->n_heads, hd, cp, sp);
    or_apply_rope(qkv + D, hkv, hd, cp, sp);
    if (tr && tr->q_rot) memcpy(tr->q_rot, qkv, sizeof(float) * (size_t)D);
    if (tr && tr->k_rot) memcpy(tr->k_rot, qkv + D, sizeof(float) * (size_t)kvd);
    /* Q to INT8 at the token's own scale; K (post-RoPE) and V to the cache at
     * the static per-layer, per-KV-head scales (design_decisions A7, B2). */
    double sq = or_quantize_int8(qkv, D, q8);
    if (tr && tr->q8) memcpy(tr->q8, q8, (size_t)D);
    if (tr && tr->q_s) tr->q_s[0] = sq;
    for (int32_t g = 0; g < hkv; g++) {
        or_quantize_static(qkv + D + g * hd, hd, m->kv_sk[layer * hkv + g], kv8);
        memcpy(k_cache + cache_row(c, layer, g, pos), kv8, (size_t)hd);
        or_quantize_static(qkv + D + kvd + g * hd, hd, m->kv_sv[layer * hkv + g], kv8);
        memcpy(v_cache + cache_row(c, layer, g, pos), kv8, (size_t)hd);
    }
    or_attention_row(c, layer, pos, q8, sq, k_cache, v_cache, m->kv_sk, m->kv_sv, att,
                     tr ? tr->scores : NULL, tr ? tr->probs : NULL, tr ? tr->pv_acc : NULL);
    if (tr && tr->attended) memcpy(tr->attended, att, sizeof(float) * (size_t)D);
    /* GI:164 O projection, GI:266 residual */
    double satt = or_quantize_int8(att, D, a8);
    linear_row(a8, satt, L->w[OR_O], L->s[OR_O], D, D, o, NULL);
    for (int32_t d = 0; d < D; d++) x[d] = x[d] + o[d];
    if (tr && tr->x_after_attn) memcpy(tr->x_after_attn, x, sizeof(float) * (size_t)D);
    /* GI:268 post-attention norm, GI:210-213 SwiGLU feed-forward, GI:270 residual */
    or_rms_norm(x, L->g_post, D, c->rms_eps, a);
    double sb = or_quantize_int8(a, D, a8);
    linear_row(a8, sb, L->w[OR_GATE], L->s[OR_GATE], F, D, gt, NULL);
    linear_row(a8, sb, L->w[OR_UP], L->s[OR_UP], F, D, up, NULL);
    for (int32_t j = 0; j < F; j++) gt[j] = or_silu(gt[j]) * up[j];
    if (tr && tr->hidden) memcpy(tr->hidden, gt, sizeof(float) * (size_t)F);
    double sh = or_quantize_int8(gt, F, a8);
    linear_row(a8, sh, L->w[OR_DOWN], L->s[OR_DOWN], D, F, o, NULL);
    for (int32_t d = 0; d < D; d++) x[d] = x[d] + o[d];
    if (tr && tr->out) memcpy(tr->out, x, sizeof(float) * (size_t)D);

    free(a); free(a8); free(qkv); free(att); free(o); free(gt); free(up); free(q8); free(kv8);
}

/* GI:463-467 final RMSNorm and INT8 LM head (per-output-channel scales,
 * design_decisions B1), GI:671 greedy argmax on the dequantized logits. */
int32_t or_lm_head_argmax(const or_model *m, const float *x, float *logits_out, float *best_logit) {
    const int32_t D = m->cfg.hidden, V = m->cfg.vocab;
    float *a = (float *)malloc(sizeof(float) * (size_t)D);
    int8_t *a8 = (int8_t *)malloc((size_t)D);
    float *logits = logits_out ? logits_out : (float *)malloc(sizeof(float) * (size_t)V);
    or_rms_norm(x, m->g_final, D, m->cfg.rms_eps, a);
    double sx = or_quantize_int8(a, D, a8);
    linear_row(a8, sx, m->lm_w, m->lm_s, V, D, logits, NULL);
    int32_t tok = or_argmax_first(logits, V);
    if (best_logit) *best_logit = logits[tok];
    if (!logits_out) free(logits);
    free(a); free(a8);
    return tok;
}

/* Several rows through one decoder layer, layer-major as GI:437-467
 * forward_mixed runs a whole sequence: row r sits at position pos[r] of the
 * sequence whose caches are k_caches[r] / v_caches[r] (rows of one sequence
 * pass the same pointers).  Each row's arithmetic is or_decode_row's, step
 * for step; the projections run as one int32 GEMM over all rows, whose exact
 * integer sums equal the per-row ones.  Every row's K/V is appended before
 * any row's attention reads the cache, and attention of a row at position p
 * visits keys 0..p only, so the rows of one prompt see exactly what
 * token-by-token decoding would have written. */
void or_decode_rows(const or_model *m, int32_t layer, int32_t rows, const int32_t *pos, float *x,
                    int8_t *const *k_caches, int8_t *const *v_caches) {
    const or_config *c = &m->cfg;
    const or_layer *L = &m->layers[layer];
    const int32_t D = c->hidden, F = c->intermediate, hd = c->head_dim;
    const int32_t hkv = c->n_kv_heads, kvd = hkv * hd, QKV = D + 2 * kvd;
    const int32_t KF = D > F ? D : F;
    float *a = (float *)malloc(sizeof(float) * (size_t)rows * D);
    int8_t *a8 = (int8_t *)malloc((size_t)rows * KF);
    double *sa = (double *)malloc(sizeof(double) * (size_t)rows);
    /* the widest projection output: Q (D), gate / up (F) */
    int32_t *acc = (int32_t *)malloc(sizeof(int32_t) * (size_t)rows * KF);
    float *qkv = (float *)malloc(sizeof(float) * (size_t)rows * QKV);
    int8_t *q8 = (int8_t *)malloc((size_t)rows * D);
    double *sq = (double *)malloc(sizeof(double) * (size_t)rows);
    float *att = (float *)malloc(sizeof(float) * (size_t)rows * D);
    float *gt = (float *)malloc(sizeof(float) * (size_t)rows * F);
    const int8_t *wqkv[3] = {L->w[OR_Q], L->w[OR_K], L->w[OR_V]};
    const float *sqkv[3] = {L->s[OR_Q], L->s[OR_K], L->s[OR_V]};
    const int32_t nqkv[3] = {D, kvd, kvd}, oqkv[3] = {0, D, D + kvd};

    /* GI:264 attention input, per row */
#pragma omp parallel for schedule(static)
    for (int32_t r = 0; r < rows; r++) {
        or_rms_norm(x + (int64_t)r * D, L->g_in, D, c->rms_eps, a + (int64_t)r * D);
        sa[r] = or_quantize_int8(a + (int64_t)r * D, D, a8 + (int64_t)r * D);
    }
    /* GI:146-148 Q/K/V projections */
    for (int i = 0; i < 3; i++) {
        or_gemm_i8(a8, wqkv[i], rows, nqkv[i], D, acc);
        for (int32_t r = 0; r < rows; r++)
            for (int32_t j = 0; j < nqkv[i]; j++)
                qkv[(int64_t)r * QKV + oqkv[i] + j] =
                    (float)acc[(int64_t)r * nqkv[i] + j] * or_dequant_mult(sa[r], (double)sqkv[i][j]);
    }
    /* GI:154 RoPE; Q to INT8 at the row's scale; K/V rows to the cache */
#pragma omp parallel for schedule(static)
    for (int32_t r = 0; r < rows; r++) {
        float *v = qkv + (int64_t)r * QKV;
        const float *cp = m->rope_cos + (int64_t)pos[r] * hd, *sp = m->rope_sin + (int64_t)pos[r] * hd;
        int8_t kv8[256];
        or_apply_rope(v, c->n_heads, hd, cp, sp);
        or_apply_rope(v + D, hkv, hd, cp, sp);
        sq[r] = or_quantize_int8(v, D, q8 + (int64_t)r * D);
        for (int32_t g = 0; g < hkv; g++) {
            or_quantize_static(v + D + g * hd, hd, m->kv_sk[layer * hkv + g], kv8);
            memcpy(k_caches[r] + cache_row(c, layer, g, pos[r]), kv8, (size_t)hd);
            or_quantize_static(v + D + kvd + g * hd, hd, m->kv_sv[layer * hkv + g], kv8);
            memcpy(v_caches[r] + cache_row(c, layer, g, pos[r]), kv8, (size_t)hd);
        }
    }
#pragma omp parallel for schedule(dynamic, 1)
    for (int32_t r = 0; r < rows; r++)
        or_attention_row(c, layer, pos[r], q8 + (int64_t)r * D, sq[r], k_caches[r], v_caches[r], m->kv_sk,
                         m->kv_sv, att + (int64_t)r * D, NULL, NULL, NULL);
    /* GI:164 O projection, GI:266 residual */
#pragma omp parallel for schedule(static)
    for (int32_t r = 0; r < rows; r++) sa[r] = or_quantize_int8(att + (int64_t)r * D, D, a8 + (int64_t)r * D);
    or_gemm_i8(a8, L->w[OR_O], rows, D, D, acc);
    for (int32_t r = 0; r < rows; r++)
        for (int32_t d = 0; d < D; d++) {
            const float o = (float)acc[(int64_t)r * D + d] * or_dequant_mult(sa[r], (double)L->s[OR_O][d]);
            x[(int64_t)r * D + d] = x[(int64_t)r * D + d] + o;
        }
    /* GI:268 post-attention norm, GI:210-213 SwiGLU, GI:270 residual */
#pragma omp parallel for schedule(static)
    for (int32_t r = 0; r < rows; r++) {
        or_rms_norm(x + (int64_t)r * D, L->g_post, D, c->rms_eps, a + (int64_t)r * D);
        sa[r] = or_quantize_int8(a + (int64_t)r * D, D, a8 + (int64_t)r * D);
    }
    or_gemm_i8(a8, L->w[OR_GATE], rows, F, D, acc);
    for (int32_t r = 0; r < rows; r++)
        for (int32_t j = 0; j < F; j++)
            gt[(int64_t)r * F + j] = (float)acc[(int64_t)r * F + j] * or_dequant_mult(sa[r], (double)L->s[OR_GATE][j]);
    or_gemm_i8(a8, L->w[OR_UP], rows, F, D, acc);
    for (int32_t r = 0; r < rows; r++)
        for (int32_t j = 0; j < F; j++) {
            const float up = (float)acc[(int64_t)r * F + j] * or_dequant_mult(sa[r], (double)L->s[OR_UP][j]);
            gt[(int64_t)r * F + j] = or_silu(gt[(int64_t)r * F + j]) * up;
        }
#pragma omp parallel for schedule(static)
    for (int32_t r = 0; r < rows; r++) sa[r] = or_quantize_int8(gt + (int64_t)r * F, F, a8 + (int64_t)r * F);
    or_gemm_i8(a8, L->w[OR_DOWN], rows, D, F, acc);
    for (int32_t r = 0; r < rows; r++)
        for (int32_t d = 0; d < D; d++) {
            const float o = (float)acc[(int64_t)r * D + d] * or_dequant_mult(sa[r], (double)L->s[OR_DOWN][d]);
            x[(int64_t)r * D + d] = x[(int64_t)r * D + d] + o;
        }
    free(a); free(a8); free(sa); free(acc); free(qkv); free(q8); free(sq); free(att); free(gt);
}

/* or_lm_head_argmax for several rows at once (one int32 GEMM over the rows):
 * tokens[r] is row r's greedy token, best_logits[r] its logit (may be NULL). */
void or_lm_head_rows(const or_model *m, int32_t rows, const float *x, int32_t *tokens, float *best_logits) {
    const int32_t D = m->cfg.hidden, V = m->cfg.vocab;
    float *a = (float *)malloc(sizeof(float) * (size_t)rows * D);
    int8_t *a8 = (int8_t *)malloc((size_t)rows * D);
    double *sa = (double *)malloc(sizeof(double) * (size_t)rows);
    int32_t *acc = (int32_t *)malloc(sizeof(int32_t) * (size_t)rows * V);
#pragma omp parallel for schedule(static)
    for (int32_t r = 0; r < rows; r++) {
        or_rms_norm(x + (int64_t)r * D, m->g_final, D, m->cfg.rms_eps, a + (int64_t)r * D);
        sa[r] = or_quantize_int8(a + (int64_t)r * D, D, a8 + (int64_t)r * D);
    }
    or_gemm_i8(a8, m->lm_w, rows, V, D, acc);
#pragma omp parallel for schedule(static)
    for (int32_t r = 0; r < rows; r++) {
        float *lg = (float *)malloc(sizeof(float) * (size_t)V);
        for (int32_t j = 0; j < V; j++)
            lg[j] = (float)acc[(int64_t)r * V + j] * or_dequant_mult(sa[r], (double)m->lm_s[j]);
        tokens[r] = or_argmax_first(lg, V);
        if (best_logits) best_logits[r] = lg[tokens[r]];
        free(lg);
    }
    free(a); free(a8); free(sa); free(acc);
}

/* Embed one token at position pos, run n_layers decoder layers (appending to
 * the cache) and return the greedy next token. */
int32_t or_forward_token(const or_model *m, int32_t token, int32_t pos, int32_t n_layers,
                         int8_t *k_cache, int8_t *v_cache, float *best_logit) {
    float *x = (float *)malloc(sizeof(float) * (size_t)m->cfg.hidden);
    or_embed(m, token, x);
    for (int32_t l = 0; l < n_layers; l++) or_decode_row(m, l, pos, x, k_cache, v_cache, NULL);
    int32_t tok = or_lm_head_argmax(m, x, NULL, best_logit);
    free(x);
    return tok;
}

/* GI:629-685 greedy generation with a KV cache: the prompt occupies positions
 * 0..n_prompt-1, then up to max_new tokens are produced, stopping after an EOS
 * token (eos_id < 0 disables).  Returns the number of generated tokens. */
int32_t or_generate(const or_model *m, const int32_t *prompt, int32_t n_prompt, int32_t max_new,
                    int32_t n_layers, int32_t eos_id, int8_t *k_cache, int8_t *v_cache,
                    int32_t *out_tokens, float *out_logits) {
    const int32_t D = m->cfg.hidden;
    if (n_prompt < 1 || max_new < 1 || n_prompt + max_new - 1 > m->cfg.max_pos) return -1;
    float *x = (float *)malloc(sizeof(float) * (size_t)D);
    for (int32_t i = 0; i < n_prompt; i++) {
        or_embed(m, prompt[i], x);
        for (int32_t l = 0; l < n_layers; l++) or_decode_row(m, l, i, x, k_cache, v_cache, NULL);
    }
    int32_t count = 0;
    for (;;) {
        float lg;
        int32_t tok = or_lm_head_argmax(m, x, NULL, &lg);
        out_tokens[count] = tok;
        if (out_logits) out_logits[count] = lg;
        count++;
        if (count >= max_new || tok == eos_id) break;
        or_embed(m, tok, x);
        for (int32_t l = 0; l < n_layers; l++)
            or_decode_row(m, l, n_prompt + count - 1, x, k_cache, v_cache, NULL);
    }
    free(x);
    return count;
}
