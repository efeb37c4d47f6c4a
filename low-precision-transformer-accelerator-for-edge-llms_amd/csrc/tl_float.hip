// tl_float.hip -- the float32 model of model/tinyllama.py (TL), the baseline
// the INT8 path is compared against by the analysis report (GI:470-626):
//   linear_f32_kernel     TL:106-110  y = x . W (+ b) (+ residual), W [K][N]
//   attention_f32_kernel  TL:122-156  scores, causal mask, softmax, P . V
// Float32 sums here run in tile order, not NumPy's, so results agree with the
// reference to float32 rounding, not bit for bit.  Not on the INT8 hot path.
#include <hip/hip_runtime.h>

#include "tl_device.h"
#include "tl_internal.h"

namespace tl {

namespace {

constexpr int kLB = 64;   // output tile 64 x 64, one 4 x 4 block per thread
constexpr int kLK = 16;   // K step staged through LDS

__global__ __launch_bounds__(256) void linear_f32_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                         const float* __restrict__ b,
                                                         const float* __restrict__ residual, int32_t m, int32_t n,
                                                         int32_t k, float* __restrict__ y) {
    __shared__ float as[kLK][kLB + 4];   // [k][row]
    __shared__ float bs[kLK][kLB];       // [k][col]
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int row0 = blockIdx.y * kLB, col0 = blockIdx.x * kLB;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;
    const int ar = tid >> 2, ak = (tid & 3) * 4;    // A: row ar, k ak..ak+3
    const int bk = tid >> 4, bc = (tid & 15) * 4;   // B: k bk, cols bc..bc+3
    for (int k0 = 0; k0 < k; k0 += kLK) {
        const int gr = row0 + ar;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int gk = k0 + ak + j;
            as[ak + j][ar] = (gr < m && gk < k) ? x[(int64_t)gr * k + gk] : 0.0f;
        }
        const int gk = k0 + bk;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int gc = col0 + bc + j;
            bs[bk][bc + j] = (gk < k && gc < n) ? w[(int64_t)gk * n + gc] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kLK; kk++) {
            float a[4], bb[4];
#pragma unroll
            for (int i = 0; i < 4; i++) a[i] = as[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; j++) bb[j] = bs[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_fmaf(a[i], bb[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = row0 + ty * 4 + i;
        if (r >= m) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int c = col0 + tx * 4 + j;
            if (c >= n) continue;
            float v = acc[i][j];
            if (b) v = v + b[c];
            const int64_t idx = (int64_t)r * n + c;
            if (residual) v = residual[idx] + v;
            y[idx] = v;
        }
    }
}

// one (query row i, query head h) per workgroup; the row's scores live in LDS
__global__ __launch_bounds__(256) void attention_f32_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                            const float* __restrict__ v, int32_t seq, int32_t n_heads,
                                                            int32_t n_kv, float scale, float* __restrict__ out,
                                                            float* __restrict__ scores, float* __restrict__ weights) {
    extern __shared__ float s[];   // [seq] scores -> exps -> probabilities, then [nblk] block sums
    __shared__ float qv[64];
    __shared__ float red[16];
    __shared__ float total_s;
    __shared__ float part[4][64];
    const int i = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = n_heads / n_kv, g = h / G;
    const int D = n_heads * kHeadDim, KVD = n_kv * kHeadDim;
    if (tid < kHeadDim) qv[tid] = q[(int64_t)i * D + h * kHeadDim + tid];
    __syncthreads();
    const int64_t srow = ((int64_t)h * seq + i) * seq;
    float mx = -INFINITY;
    for (int t = tid; t < seq; t += blockDim.x) {
        float val = -1e9f;   // TL:90-91 causal mask value
        if (t <= i) {
            const float* kr = k + (int64_t)t * KVD + g * kHeadDim;
            float acc = 0.0f;
#pragma unroll 16
            for (int d = 0; d < kHeadDim; d++) acc = __builtin_fmaf(qv[d], kr[d], acc);
            val = acc * scale;
        }
        s[t] = val;
        if (scores) scores[srow + t] = val;
        mx = fmaxf(mx, val);
    }
    const float m = block_max(mx, red);
    const int nblk = (seq + 63) >> 6;
    float* bsum = s + seq;
    for (int bi = wave; bi < nblk; bi += blockDim.x >> 6) {
        const int t = bi * 64 + lane;
        float e = 0.0f;
        if (t < seq) {
            e = tl_expf(s[t] - m);
            s[t] = e;
        }
        const float bsv = wave_butterfly_sum(e);
        if (lane == 0) bsum[bi] = bsv;
    }
    __syncthreads();
    if (tid == 0) {
        float tot = 0.0f;
        for (int bi = 0; bi < nblk; bi++) tot = tot + bsum[bi];
        total_s = tot;
    }
    __syncthreads();
    const float tot = total_s;
    for (int t = tid; t < seq; t += blockDim.x) {
        const float p = __fdiv_rn(s[t], tot);
        s[t] = p;
        if (weights) weights[srow + t] = p;
    }
    __syncthreads();
    // keys past i have probability 0 exactly and are skipped
    float acc = 0.0f;
    for (int t = wave; t <= i; t += 4) acc = __builtin_fmaf(s[t], v[(int64_t)t * KVD + g * kHeadDim + lane], acc);
    part[wave][lane] = acc;
    __syncthreads();
    if (tid < kHeadDim)
        out[(int64_t)i * D + h * kHeadDim + tid] = ((part[0][tid] + part[1][tid]) + part[2][tid]) + part[3][tid];
}

}  // namespace

hipError_t launch_linear_f32(hipStream_t s, const float* x, const float* w, const float* b, const float* residual,
                             int32_t m, int32_t n, int32_t k, float* y) {
    if (m <= 0 || n <= 0) return hipSuccess;
    const dim3 grid((n + kLB - 1) / kLB, (m + kLB - 1) / kLB);
    TL_KLAUNCH(linear_f32_kernel, grid, dim3(256), 0, s, x, w, b, residual, m, n, k, y);
    return hipGetLastError();
}

hipError_t launch_attention_f32(hipStream_t s, const float* q, const float* k, const float* v, int32_t seq,
                                int32_t n_heads, int32_t n_kv, float scale, float* out, float* scores,
                                float* weights) {
    if (seq <= 0) return hipSuccess;
    const size_t lds = sizeof(float) * ((size_t)seq + (seq + 63) / 64);
    TL_KLAUNCH(attention_f32_kernel, dim3(seq, n_heads), dim3(256), lds, s, q, k, v, seq, n_heads, n_kv, scale, out,
               scores, weights);
    return hipGetLastError();
}

}  // namespace tl
