// The softmax exponential of the GPU kernels (csrc/tl_device.h,
// tl_expf_nonpos) against the exponential it replaces there (tl_expf_sel,
// the oracle's tl_expf without branches), bit for bit over every float x in
// [-90, -0]: the same Cody-Waite reduction and degree-7 polynomial, but no
// clamp of x to [-80, 80] before the reduction and 2^k applied by ldexp
// instead of a multiply by the power of two built in the exponent field.
// Below -80 both return 0 by the final select; at or above -80, k lies in
// [-116, 0], where p 2^k is a normal float.  Prints the counts; exits 1 on a
// mismatch.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static inline float fbits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t bitsf(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float poly(float x, float* kfo) {
    const float log2e = 0x1.715476p+0f, c1 = 0x1.63p-1f, c2 = -0x1.bd0106p-13f;
    const float kf = rintf(x * log2e);
    float r = fmaf(-kf, c1, x);
    r = fmaf(-kf, c2, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    *kfo = kf;
    return p;
}

static float exp_sel(float x) {   // clamp, reduce, scale by the exponent-field power of two, select
    float kf;
    const float p = poly(fminf(fmaxf(x, -80.0f), 80.0f), &kf);
    const float e = p * fbits((uint32_t)((int)kf + 127) << 23);
    return x >= -80.0f ? e : 0.0f;
}

static float exp_nonpos(float x) {   // no clamp, ldexp, select
    float kf;
    const float p = poly(x, &kf);
    // the GPU's conversion saturates for the huge k of x far below -80; C's
    // is undefined there, so the exponent is bounded first (the value is
    // discarded by the select either way)
    const float e = ldexpf(p, (int)fmaxf(kf, -1000.0f));
    return x >= -80.0f ? e : 0.0f;
}

int main(void) {
    const uint32_t lo = 0x80000000u, hi = bitsf(-90.0f);
    long n = 0, bad = 0;
#pragma omp parallel for reduction(+ : n, bad) schedule(static)
    for (int64_t u = lo; u <= (int64_t)hi; u++) {
        const float x = fbits((uint32_t)u);
        n++;
        if (bitsf(exp_sel(x)) != bitsf(exp_nonpos(x))) bad++;
    }
    printf("floats in [-90, -0]: %ld, mismatches %ld\n", n, bad);
    return bad != 0;
}
