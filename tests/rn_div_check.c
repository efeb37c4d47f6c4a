// The row-uniform division of the GPU quantizers (csrc/tl_device.h,
// rn_div_fast): y = RN(1/b), q0 = RN(a y), two FMA residual corrections
// q <- RN(q + RN(a - b q) y).  Checked against RN(a/b) formed as the float64
// quotient rounded to float32 (double rounding is innocuous for division
// when 53 >= 2 * 24 + 2).  Cases: random significands over 121 binades of b,
// quotients next to half-integers and to float32 midpoints, and divisors with
// extreme significands.  Prints the mismatch counts; exits 1 on any mismatch.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
static uint64_t s = 88172645463325252ull;
static inline uint64_t rnd(void) { s ^= s << 13; s ^= s >> 7; s ^= s << 17; return s; }
static inline float fbits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t bitsf(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float q2div(float a, float b, float y) {
    float q0 = a * y;
    float r0 = fmaf(-b, q0, a);
    float q1 = fmaf(r0, y, q0);
    float r1 = fmaf(-b, q1, a);
    return fmaf(r1, y, q1);
}
static long bad = 0, n = 0, badint = 0;
static void check(float a, float b) {
    float y = (float)(1.0 / (double)b);   // RN(1/b) (double rounding innocuous)
    float want = (float)((double)a / (double)b);
    float got = q2div(a, b, y);
    n++;
    if (bitsf(got) != bitsf(want) && !(got == 0 && want == 0)) {
        if (bad < 10) printf("mismatch a=%a b=%a got %a want %a\n", a, b, got, want);
        bad++;
    }
    if (rintf(got) != rintf(want)) badint++;
}
int main(int argc, char** argv) {
    long N = argc > 1 ? atol(argv[1]) : 100000000L;
    // 1) random significands, b in [2^-60, 2^60], |a/b| <= 2^8
    for (long i = 0; i < N; i++) {
        uint32_t mb = rnd() & 0x7FFFFF, ma = rnd() & 0x7FFFFF;
        int eb = (int)(rnd() % 121) - 60;
        float b = ldexpf(fbits(0x3F800000u | mb), eb);
        int ea = eb + (int)(rnd() % 40) - 30;
        float a = ldexpf(fbits(0x3F800000u | ma), ea);
        if (rnd() & 1) a = -a;
        check(a, b);
    }
    // 2) quotients near half-integers and near float midpoints
    for (long i = 0; i < N / 4; i++) {
        uint32_t mb = rnd() & 0x7FFFFF;
        int eb = (int)(rnd() % 41) - 20;
        float b = ldexpf(fbits(0x3F800000u | mb), eb);
        double t;
        if (i & 1) t = (double)((int)(rnd() % 255) - 127) + 0.5;
        else {   // midpoint between two floats of random magnitude <= 128
            float f = ldexpf(fbits(0x3F800000u | (rnd() & 0x7FFFFF)), (int)(rnd() % 30) - 22);
            t = ((double)f + (double)nextafterf(f, INFINITY)) * 0.5;
        }
        float a0 = (float)(t * (double)b);
        float a = a0;
        for (int k = 0; k < 3; k++) a = nextafterf(a, -INFINITY);
        for (int k = 0; k < 7; k++) { check(a, b); a = nextafterf(a, INFINITY); }
    }
    // 3) divisors with extreme significands (all ones, one, one + ulp)
    uint32_t sig[] = {0x000000, 0x000001, 0x7FFFFF, 0x7FFFFE, 0x400000, 0x3FFFFF};
    for (int si = 0; si < 6; si++)
        for (long i = 0; i < N / 10; i++) {
            float b = ldexpf(fbits(0x3F800000u | sig[si]), (int)(rnd() % 21) - 10);
            float a = ldexpf(fbits(0x3F800000u | (rnd() & 0x7FFFFF)), (int)(rnd() % 30) - 20);
            check(a, b);
            check(nextafterf(a, 0), b);
        }
    printf("checked %ld, float mismatches %ld, rint mismatches %ld\n", n, bad, badint);
    return bad != 0;
}
