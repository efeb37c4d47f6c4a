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

// INT8 row into LDS: chunk c of thread t holds elements 4 (256 c + t) .. +3;
// bytes beyond K stay zero (they meet padded weight lanes)
template <bool FAST, int KCH>
TL_DEV void quant_row(const float4 (&v)[KCH], int K, const RnDiv& dv, int8_t* xs8) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int c = 0; c < KCH; c++) {
        const int idx = c * kNT + tid;
        ((unsigned*)xs8)[idx] = idx * 4 < K ? quant4<FAST>(v[c], dv) : 0u;
    }
}

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
    const RnDiv dv = rn_div_prep((float)s);
    // |x| <= max |x| = 127 b (1 + 2^-24) keeps every x y finite
    if (dv.fast) quant_row<true, KCH>(xv, K, dv, xs8);
    else quant_row<false, KCH>(xv, K, dv, xs8);
    if (tid == 0) *xscale = s;
    __syncthreads();
}

// sum of squares of a row through LDS in NumPy's pairwise order (plan's
// perfect tree); every thread gets the sum
template <int KCH>
TL_DEV float prologue_sumsq(const float4 (&xv)[KCH], int K, PwPlan plan, float* sq, float* part, float* red) {
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
    return red[8];
}

// ---------------------------------------------------------------------------
// NumPy's pairwise sum of squares of a 2048-element row (16 leaves of 128)
// with one barrier.  Wavefront w holds leaves 2w, 2w+1 (chunk 0) and
// 8+2w, 9+2w (chunk 1) in its float4 registers; it transposes their squares
// through its own 512 floats of LDS (element e of local leaf ll at
// 128 ll + (e ^ 8 ll), so the strided reads of 32 lanes hit 32 banks), lane
// 8 ll + r sums accumulator r of local leaf ll in order, lane pairs 1, 2, 4
// apart combine a leaf's accumulators and lane pairs 8 apart the two leaves
// of a chunk.  The eight pair sums meet in LDS and every thread finishes the
// tree ((P0+P1)+(P2+P3))+((P4+P5)+(P6+P7)).  sq needs 2048 floats, part 8.
// ---------------------------------------------------------------------------

TL_DEV bool pw_by_waves(PwPlan plan, int K) {
    return plan.leaf_len == 128 && plan.n_leaves == 16 && K == 2048;
}

TL_DEV float pw_sumsq_2048(const float4 (&xv)[2], float* sq, float* part) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float* mine = sq + wave * 512;
#pragma unroll
    for (int c = 0; c < 2; c++) {
        float4 q;
        q.x = xv[c].x * xv[c].x;
        q.y = xv[c].y * xv[c].y;
        q.z = xv[c].z * xv[c].z;
        q.w = xv[c].w * xv[c].w;
        const int ll = 2 * c + (lane >> 5);
        *(float4*)(mine + 128 * ll + ((4 * (lane & 31)) ^ (8 * ll))) = q;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wavefront's stores are in LDS
    __builtin_amdgcn_wave_barrier();
    const int ll = (lane & 31) >> 3;
    const float* a = mine + 128 * ll;
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; u++) v[u] = a[((lane & 7) + 8 * u) ^ (8 * ll)];
    float r = v[0];
#pragma unroll
    for (int u = 1; u < 16; u++) r = r + v[u];
    r = r + lane_xor<1>(r);
    r = r + lane_xor<2>(r);
    r = r + lane_xor<4>(r);   // local leaf ll = (lane & 31) >> 3
    r = r + lane_xor<8>(r);   // lane 0: leaves 2w + 2w+1, lane 16: leaves 8+2w + 9+2w
    if (lane == 0) part[wave] = r;
    if (lane == 16) part[4 + wave] = r;
    __syncthreads();
    const float4 p0 = *(const float4*)part, p1 = *(const float4*)(part + 4);
    return ((p0.x + p0.y) + (p0.z + p0.w)) + ((p1.x + p1.y) + (p1.z + p1.w));
}

template <int KCH>
TL_DEV void prologue_rmsnorm(const float4 (&xv)[KCH], const float4 (&gv)[KCH], int K, float eps, PwPlan plan,
                             float* sq, float* part, int8_t* xs8, float* red, double* xscale) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float total;
    if constexpr (KCH == 2) {
        if (pw_by_waves(plan, K)) {
            total = pw_sumsq_2048(xv, sq, part);
        } else {
            total = prologue_sumsq<KCH>(xv, K, plan, sq, part, red);
        }
    } else {
        total = prologue_sumsq<KCH>(xv, K, plan, sq, part, red);
    }
    const float var = __fdiv_rn(total, (float)K);
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
    const RnDiv dv = rn_div_prep((float)s);
    // |x| <= max |x| = 127 b (1 + 2^-24) keeps every x y finite
    if (dv.fast) quant_row<true, KCH>(av, K, dv, xs8);
    else quant_row<false, KCH>(av, K, dv, xs8);
    if (tid == 0) *xscale = s;
    __syncthreads();
}

}  // namespace tl
