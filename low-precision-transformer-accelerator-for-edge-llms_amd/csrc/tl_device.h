// tl_device.h -- device-side arithmetic shared by every kernel file.  Each
// helper is the exact operation sequence the CPU oracle (oracle/tl_oracle.c)
// performs, so kernels built from them agree with it bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "tl_internal.h"

namespace tl {

#define TL_DEV __device__ __forceinline__

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// scalar helpers
// ---------------------------------------------------------------------------

// exp(x): Cody-Waite reduction x = k ln2 + r (ln2 = 355/512 + remainder),
// degree-7 Taylor polynomial (1/n! in float32) in Horner form with explicit
// fused multiply-adds, times 2^k from the exponent field.  x < -80 -> 0.
TL_DEV float tl_expf(float x) {
    if (!(x >= -80.0f)) return 0.0f;
    if (x > 80.0f) x = 80.0f;
    const float log2e = 0x1.715476p+0f;
    const float c1 = 0x1.63p-1f;
    const float c2 = -0x1.bd0106p-13f;
    float kf = __builtin_rintf(x * log2e);
    float r = __builtin_fmaf(-kf, c1, x);
    r = __builtin_fmaf(-kf, c2, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    int k = (int)kf;
    return p * __int_as_float((k + 127) << 23);
}

// tl_expf without branches, the same value for every input: the argument is
// clamped to [-80, 80] before the reduction and the result is 0 below -80
// (and for NaN), as in tl_expf
TL_DEV float tl_expf_sel(float x) {
    const float xc = fminf(fmaxf(x, -80.0f), 80.0f);
    const float log2e = 0x1.715476p+0f;
    const float c1 = 0x1.63p-1f;
    const float c2 = -0x1.bd0106p-13f;
    float kf = __builtin_rintf(xc * log2e);
    float r = __builtin_fmaf(-kf, c1, xc);
    r = __builtin_fmaf(-kf, c2, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int k = (int)kf;
    const float e = p * __int_as_float((k + 127) << 23);
    return x >= -80.0f ? e : 0.0f;
}

// SiLU, TL:159-161: x / (1 + exp(-clip(x, -60, 60)))
TL_DEV float tl_silu(float x) {
    float c = x < -60.0f ? -60.0f : (x > 60.0f ? 60.0f : x);
    return __fdiv_rn(x, 1.0f + tl_expf(-c));
}

TL_DEV int8_t sat_i8(float v) {
    v = v > 127.0f ? 127.0f : v;
    v = v < -127.0f ? -127.0f : v;
    return (int8_t)(int)v;
}

// GI:36-42 scale: max|x| / 127 in float64, 1.0 for an all-zero tensor
TL_DEV double quant_scale(float mx) { return mx != 0.0f ? (double)mx / 127.0 : 1.0; }

// GI:45-46 dequantization multiplier, formed in float64, rounded once
TL_DEV float deq_mult(double sx, float sw) { return (float)(sx * (double)sw); }

// 64-bit argmax key: order-preserving float bits above, (~index) below, so the
// maximum key is the largest logit with the lowest index (B4 tie-break).
TL_DEV unsigned long long argmax_key(float v, int32_t idx) {
    if (v == 0.0f) v = 0.0f;  // -0 and +0 compare equal in np.argmax
    unsigned u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned)idx);
}

TL_DEV float key_logit(unsigned long long key) {
    unsigned u = (unsigned)(key >> 32);
    u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
    return __uint_as_float(u);
}

TL_DEV int32_t key_index(unsigned long long key) {
    return (int32_t)(0xFFFFFFFFu - (unsigned)(key & 0xFFFFFFFFull));
}

TL_DEV int wave_sum_i32(int v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

TL_DEV float wave_max_f32(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// the fixed 64-wide butterfly (same tree as or_block_sum64)
TL_DEV float wave_butterfly_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off);
    return v;
}

TL_DEV unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        unsigned lo = __shfl_xor((unsigned)(v & 0xFFFFFFFFull), off);
        unsigned hi = __shfl_xor((unsigned)(v >> 32), off);
        unsigned long long o = ((unsigned long long)hi << 32) | lo;
        v = o > v ? o : v;
    }
    return v;
}

// 128-bit loads that stay 128-bit: weights stream through once (non-temporal)
TL_DEV v4i ld_nt16(const int8_t* p) { return __builtin_nontemporal_load((const v4i*)p); }
TL_DEV v4i ld16(const int8_t* p) { return *(const v4i*)p; }

TL_DEV int sdot4v(v4i a, v4i b, int acc) {
    acc = __builtin_amdgcn_sdot4(a[0], b[0], acc, false);
    acc = __builtin_amdgcn_sdot4(a[1], b[1], acc, false);
    acc = __builtin_amdgcn_sdot4(a[2], b[2], acc, false);
    acc = __builtin_amdgcn_sdot4(a[3], b[3], acc, false);
    return acc;
}

TL_DEV int sdot4x4(int4 a, int4 b, int acc) {
    acc = __builtin_amdgcn_sdot4(a.x, b.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a.y, b.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, b.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, b.w, acc, false);
    return acc;
}

// v[0] + v[1] + ... + v[n-1] added in index order, starting from 0 (the
// softmax denominator over block sums); up to 32 values are read before the
// first add, so the chain costs one LDS latency instead of n
TL_DEV float ordered_sum(const float* v, int n) {
    float t = 0.0f;
    if (n <= 32) {
        float r[32];
#pragma unroll
        for (int i = 0; i < 32; i++) r[i] = v[i < n ? i : 0];
#pragma unroll
        for (int i = 0; i < 32; i++)
            if (i < n) t = t + r[i];
        return t;
    }
    for (int i = 0; i < n; i++) t = t + v[i];
    return t;
}

// block-wide max of a non-negative float (all threads get the result)
TL_DEV float block_max(float v, float* red /* >= 16 floats */) {
    v = wave_max_f32(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
    for (int i = 1; i < nw; i++) m = fmaxf(m, red[i]);
    return m;
}

// NumPy pairwise sum of sq[0 .. plan.leaf_len*plan.n_leaves) (a perfect
// tree): 8 strided accumulators per leaf, ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7))
// per leaf, then leaves combined pairwise level by level.  scr needs
// 10 * n_leaves floats.  Returns the sum in every thread.
TL_DEV float block_pairwise_sum(const float* sq, PwPlan plan, float* scr) {
    const int tid = threadIdx.x, nt = blockDim.x;
    const int L = plan.n_leaves, len = plan.leaf_len;
    float* part = scr;           // [8 L]
    float* lv0 = scr + 8 * L;    // [L]
    float* lv1 = lv0 + L;        // [L]
    for (int idx = tid; idx < 8 * L; idx += nt) {
        // leaf_len <= 128: at most 16 steps, read before the in-order sum
        const float* a = sq + (idx >> 3) * len + (idx & 7);
        float v[16];
#pragma unroll
        for (int t = 0; t < 16; t++) v[t] = a[min(8 * t, len - 8)];
        float r = v[0];
#pragma unroll
        for (int t = 1; t < 16; t++)
            if (8 * t < len) r = r + v[t];
        part[idx] = r;
    }
    __syncthreads();
    for (int leaf = tid; leaf < L; leaf += nt) {
        const float* r = part + 8 * leaf;
        lv0[leaf] = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    }
    __syncthreads();
    float* cur = lv0;
    float* nxt = lv1;
    for (int w = L; w > 1; w >>= 1) {
        for (int i = tid; i < (w >> 1); i += nt) nxt[i] = cur[2 * i] + cur[2 * i + 1];
        __syncthreads();
        float* t = cur; cur = nxt; nxt = t;
    }
    return cur[0];
}

}  // namespace tl
