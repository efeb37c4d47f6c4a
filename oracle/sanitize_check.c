/*
 * sanitize_check.c -- TEST INFRASTRUCTURE ONLY.  Runs the oracle's composed
 * path on a small seeded model under AddressSanitizer and
 * UndefinedBehaviorSanitizer (oracle/Makefile, target `sanitize`): any heap
 * overflow, use of freed memory or undefined arithmetic in tl_oracle.c stops
 * the program with a report.  Geometries include hidden > intermediate (the
 * projection accumulators must hold the widest output) and the reverse.
 * Also checks that the layer-major multi-row forms equal the per-row ones
 * bit for bit, as tests/test_oracle_pins.py does through Python.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tl_oracle.h"

static uint64_t g_state = 0x9E3779B97F4A7C15ull;

static uint32_t rnd(void) {
    g_state = g_state * 6364136223846793005ull + 1442695040888963407ull;
    return (uint32_t)(g_state >> 33);
}

static float rnd_f(float lo, float hi) { return lo + (hi - lo) * (float)(rnd() & 0xFFFFFF) / (float)0x1000000; }

static int8_t *rand_i8(size_t n) {
    int8_t *p = (int8_t *)malloc(n);
    for (size_t i = 0; i < n; i++) p[i] = (int8_t)((int)(rnd() % 255) - 127);
    return p;
}

static float *rand_f(size_t n, float lo, float hi) {
    float *p = (float *)malloc(sizeof(float) * n);
    for (size_t i = 0; i < n; i++) p[i] = rnd_f(lo, hi);
    return p;
}

static int run(int32_t hidden, int32_t inter, int32_t heads, int32_t kv_heads) {
    or_config c = {hidden, inter, 2, heads, kv_heads, 64, 96, 40, 1e-5f, 10000.0f};
    const int32_t D = c.hidden, F = c.intermediate, hd = c.head_dim, kvd = c.n_kv_heads * hd;
    const int32_t nout[OR_NW] = {D, kvd, kvd, D, F, F, D}, nin[OR_NW] = {D, D, D, D, D, D, F};
    or_layer layers[2];
    for (int l = 0; l < c.n_layers; l++) {
        for (int t = 0; t < OR_NW; t++) {
            layers[l].w[t] = rand_i8((size_t)nout[t] * nin[t]);
            layers[l].s[t] = rand_f((size_t)nout[t], 1e-4f, 2e-3f);
        }
        layers[l].g_in = rand_f((size_t)D, 0.9f, 1.1f);
        layers[l].g_post = rand_f((size_t)D, 0.9f, 1.1f);
    }
    float *cs = (float *)malloc(sizeof(float) * (size_t)c.max_pos * hd);
    float *sn = (float *)malloc(sizeof(float) * (size_t)c.max_pos * hd);
    for (int p = 0; p < c.max_pos; p++)
        for (int d = 0; d < hd; d++) {
            const float a = (float)p * powf(c.rope_theta, -(float)(2 * (d % (hd / 2))) / (float)hd);
            cs[p * hd + d] = cosf(a);
            sn[p * hd + d] = sinf(a);
        }
    or_model m = {c, layers, rand_i8((size_t)c.vocab * D), rand_f((size_t)c.vocab, 1e-4f, 2e-3f),
                  rand_f((size_t)D, 0.9f, 1.1f), rand_i8((size_t)c.vocab * D), rand_f((size_t)c.vocab, 1e-3f, 1e-2f),
                  cs, sn, rand_f((size_t)c.n_layers * c.n_kv_heads, 0.02f, 0.08f),
                  rand_f((size_t)c.n_layers * c.n_kv_heads, 0.02f, 0.08f)};
    const size_t cache = (size_t)c.n_layers * c.n_kv_heads * c.max_pos * hd;
    enum { ROWS = 3 };
    int8_t *k1[ROWS], *v1[ROWS], *kr[ROWS], *vr[ROWS];
    float *x1 = (float *)malloc(sizeof(float) * (size_t)ROWS * D);
    float *xr = (float *)malloc(sizeof(float) * (size_t)ROWS * D);
    int32_t pos[ROWS] = {0, 7, c.max_pos - 1};
    for (int r = 0; r < ROWS; r++) {
        k1[r] = rand_i8(cache);
        v1[r] = rand_i8(cache);
        kr[r] = (int8_t *)malloc(cache);
        vr[r] = (int8_t *)malloc(cache);
        memcpy(kr[r], k1[r], cache);
        memcpy(vr[r], v1[r], cache);
        or_embed(&m, (int32_t)(rnd() % (uint32_t)c.vocab), x1 + (size_t)r * D);
    }
    memcpy(xr, x1, sizeof(float) * (size_t)ROWS * D);
    for (int l = 0; l < c.n_layers; l++) {
        for (int r = 0; r < ROWS; r++) or_decode_row(&m, l, pos[r], x1 + (size_t)r * D, k1[r], v1[r], NULL);
        or_decode_rows(&m, l, ROWS, pos, xr, kr, vr);
    }
    int bad = memcmp(x1, xr, sizeof(float) * (size_t)ROWS * D) != 0;
    for (int r = 0; r < ROWS; r++) bad |= memcmp(k1[r], kr[r], cache) != 0 || memcmp(v1[r], vr[r], cache) != 0;
    int32_t ids[ROWS];
    float lg[ROWS];
    or_lm_head_rows(&m, ROWS, xr, ids, lg);
    for (int r = 0; r < ROWS; r++) {
        float best = 0.0f;
        bad |= or_lm_head_argmax(&m, x1 + (size_t)r * D, NULL, &best) != ids[r] || best != lg[r];
    }
    printf("hidden %d intermediate %d: %s\n", D, F, bad ? "MISMATCH" : "ok");
    for (int r = 0; r < ROWS; r++) {
        free(k1[r]); free(v1[r]); free(kr[r]); free(vr[r]);
    }
    free(x1); free(xr); free(cs); free(sn);
    for (int l = 0; l < c.n_layers; l++) {
        for (int t = 0; t < OR_NW; t++) {
            free((void *)layers[l].w[t]);
            free((void *)layers[l].s[t]);
        }
        free((void *)layers[l].g_in);
        free((void *)layers[l].g_post);
    }
    free((void *)m.lm_w); free((void *)m.lm_s); free((void *)m.g_final); free((void *)m.emb);
    free((void *)m.emb_s); free((void *)m.kv_sk); free((void *)m.kv_sv);
    return bad;
}

int main(void) {
    int bad = 0;
    bad |= run(256, 128, 4, 2);    /* hidden > intermediate */
    bad |= run(128, 384, 2, 1);    /* intermediate > hidden */
    return bad;
}
