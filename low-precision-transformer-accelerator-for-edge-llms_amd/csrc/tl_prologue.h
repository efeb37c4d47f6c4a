// tl_prologue.h -- activation prologues of the decode GEMVs, shared by the
// fused per-layer kernels and the persistent decode kernel: an f32 row (K
// elements, 4 per float4 chunk, chunk c of thread t holding elements
// 4 (256 c + t) .. +3) becomes an INT8 row in LDS (natural byte order) and its
// float64 scale.  RMSNorm follows TL:45-50 with NumPy's pairwise summation
// order; quantization follows GI:36-42 per row.
#pragma once

#include "tl_device.h"
#include "tl_internal.h"

namespace tl {

constexpr int kNT = 256;   // threads per workgroup of the fused GEMV
constexpr int kNW = kNT / 64;

// ---------------------------------------------------------------------------
// activation prologues: f32 row (K elements, 4 per float4 chunk) -> INT8 row
// in LDS (natural byte order) + its float64 scale
// ---------------------------------------------------------------------------
template <int KCH>
TL_DEV void prologue_quant(const float4 (&xv)[KCH], int K, int8_t* xs8, float* red, double* xscale) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float mx = 0.0f;
#pragma unroll
    for (int c = 0; c < KCH; c++) {
        if ((c * kNT + tid) * 4 < K) {
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(xv[c].x), fabsf(xv[c].y)), fmaxf(fabsf(xv[c].z), fabsf(xv[c].w))));
        }
    }
    mx = wave_max_f32(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const double s = quant_scale(mx);
    const float sf = (float)s;
#pragma unroll
    for (int c = 0; c < KCH; c++) {
        const int idx = c * kNT + tid;
        unsigned word = 0;  // bytes beyond K stay zero: they meet padded weight lanes
        if (idx * 4 < K) {
            const unsigned b0 = (uint8_t)sat_i8(__builtin_rintf(__fdiv_rn(xv[c].x, sf)));
            const unsigned b1 = (uint8_t)sat_i8(__builtin_rintf(__fdiv_rn(xv[c].y, sf)));
            const unsigned b2 = (uint8_t)sat_i8(__builtin_rintf(__fdiv_rn(xv[c].z, sf)));
            const unsigned b3 = (uint8_t)sat_i8(__builtin_rintf(__fdiv_rn(xv[c].w, sf)));
            word = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
        }
        ((unsigned*)xs8)[idx] = word;
    }
    if (tid == 0) *xscale = s;
    __syncthreads();
}

template <int KCH>
TL_DEV void prologue_rmsnorm(const float4 (&xv)[KCH], const float4 (&gv)[KCH], int K, float eps, PwPlan plan,
                             float* sq, float* part, int8_t* xs8, float* red, double* xscale) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int c = 0; c < KCH; c++) {
        const int idx = c * kNT + tid;
        if (idx * 4 < K) {
            float4 q;
            q.x = xv[c].x * xv[c].x;
            q.y = xv[c].y * xv[c].y;
            q.z = xv[c].z * xv[c].z;
            q.w = xv[c].w * xv[c].w;
            ((float4*)sq)[idx] = q;
        }
    }
    __syncthreads();
    // NumPy pairwise tree: eight strided accumulators per leaf (leaf_len <=
    // 128: at most 16 steps; all reads are issued before the in-order sum,
    // steps past the leaf read an in-bounds stand-in and are not added) ...
    const int L = plan.n_leaves, len = plan.leaf_len;
    for (int p = tid; p < 8 * L; p += kNT) {
        const float* a = sq + (p >> 3) * len + (p & 7);
        float v[16];
#pragma unroll
        for (int t = 0; t < 16; t++) v[t] = a[min(8 * t, len - 8)];
        float r = v[0];
#pragma unroll
        for (int t = 1; t < 16; t++)
            if (8 * t < len) r = r + v[t];
        part[p] = r;
    }
    __syncthreads();
    // ... combined per leaf, then leaves pairwise across lanes of wave 0
    if (wave == 0) {
        float v = 0.0f;
        if (lane < L) {
            const float* r = part + 8 * lane;
            v = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        }
        for (int off = 1; off < L; off <<= 1) v = v + lane_xor_rt(v, off);
        if (lane == 0) red[8] = v;
    }
    __syncthreads();
    const float var = __fdiv_rn(red[8], (float)K);
    const float inv = __fdiv_rn(1.0f, __builtin_sqrtf(var + eps));
    float4 av[KCH];
    float mx = 0.0f;
#pragma unroll
    for (int c = 0; c < KCH; c++) {
        if ((c * kNT + tid) * 4 < K) {
            av[c].x = (xv[c].x * inv) * gv[c].x;
            av[c].y = (xv[c].y * inv) * gv[c].y;
            av[c].z = (xv[c].z * inv) * gv[c].z;
            av[c].w = (xv[c].w * inv) * gv[c].w;
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(av[c].x), fabsf(av[c].y)), fmaxf(fabsf(av[c].z), fabsf(av[c].w))));
        }
    }
    mx = wave_max_f32(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const double s = quant_scale(mx);
    const float sf = (float)s;
#pragma unroll
    for (int c = 0; c < KCH; c++) {
        const int idx = c * kNT + tid;
        unsigned word = 0;
        if (idx * 4 < K) {
            const unsigned b0 = (uint8_t)sat_i8(__builtin_rintf(__fdiv_rn(av[c].x, sf)));
            const unsigned b1 = (uint8_t)sat_i8(__builtin_rintf(__fdiv_rn(av[c].y, sf)));
            const unsigned b2 = (uint8_t)sat_i8(__builtin_rintf(__fdiv_rn(av[c].z, sf)));
            const unsigned b3 = (uint8_t)sat_i8(__builtin_rintf(__fdiv_rn(av[c].w, sf)));
            word = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
        }
        ((unsigned*)xs8)[idx] = word;
    }
    if (tid == 0) *xscale = s;
    __syncthreads();
}

}  // namespace tl
